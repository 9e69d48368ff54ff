"""GPU parity: backward passes and losses vs the CPU oracle.

The oracle restates the autograd closures of backend.rs (relu/gelu/softmax/
matmul/add/sub backward, cross entropy and MSE with their backward).
Tolerances:
  * elementwise backward: 1e-5 relative, plus the absolute error the
    reference's f32 formula itself has where its terms cancel (GELU's
    derivative near its zero and at |x| ~ 8), scaled by |grad_out|;
  * softmax backward and the losses (reductions): 1e-4 relative, with the
    absolute part of a row reduction scaled by y * sum|dy * y|;
  * matmul backward: the matmul bound, 2e-3 relative + 1e-4 * max|C|;
  * the broadcast gradient on small-integer data: bit-exact (every partial
    sum is exact, so any summation order gives the oracle's bits).
Every reduction is deterministic: a second call gives the same bits.
"""
import numpy as np
import pytest

import oracle
from conftest import assert_close, rng

pytestmark = pytest.mark.gpu


# ---- elementwise backward ------------------------------------------------

@pytest.mark.parametrize("n", [0, 1, 3, 17, 4096, 1 << 20])
def test_relu_backward_exact(hip, n):
    g = rng(n + 1)
    x = g.standard_normal(n).astype(np.float32)
    go = g.standard_normal(n).astype(np.float32)
    got = hip.relu_backward(hip.tensor(x), hip.tensor(go)).numpy()
    assert np.array_equal(got, oracle.relu_backward(x, go))


@pytest.mark.parametrize("n", [1, 5, 4099, 1 << 20])
def test_gelu_backward(hip, n):
    g = rng(n + 2)
    x = (g.standard_normal(n) * 3).astype(np.float32)
    go = g.standard_normal(n).astype(np.float32)
    got = hip.gelu_backward(hip.tensor(x), hip.tensor(go)).numpy()
    want = oracle.gelu_backward(x, go)
    bound = 1e-5 * np.abs(want) + np.where(np.abs(x) < 3, 2e-7, 3e-6) * np.abs(go) + 1e-30
    assert np.all(np.abs(got - want) <= bound)


def test_elementwise_backward_shape_errors(hip):
    with pytest.raises(hip.CloveError):
        hip.relu_backward(hip.tensor(np.ones(4, np.float32)), hip.tensor(np.ones(5, np.float32)))


# ---- softmax backward ----------------------------------------------------

def softmax_bw_check(got, y, dy, what):
    want = oracle.softmax_backward(y, dy)
    # error of the row sum s (summed in another order) reaches dx as y * ds
    ds = 1e-5 * np.sum(np.abs(dy * y), axis=-1, keepdims=True)
    bound = 1e-4 * np.abs(want) + y * ds + 1e-12
    err = np.abs(got - want)
    assert np.all(err <= bound), f"{what}: max excess {np.max(err - bound):.3e}"


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 3), (5, 17), (64, 256), (7, 4100),
                                       (33, 8192), (2, 8200), (100, 10)])
def test_softmax_backward_shapes(hip, rows, cols):
    g = rng(rows * 31 + cols)
    y = oracle.softmax(g.normal(0, 2, (rows, cols)).astype(np.float32))
    dy = g.standard_normal((rows, cols)).astype(np.float32)
    got = hip.softmax_backward(hip.tensor(y), hip.tensor(dy)).numpy()
    softmax_bw_check(got, y, dy, f"softmax backward {rows}x{cols}")


def test_softmax_backward_config3_full(hip):
    """The config-3 shape: [8192, 4096], y = softmax(normal(0, 2))."""
    g = rng(2)
    x = g.normal(0, 2, (8192, 4096)).astype(np.float32)
    dy = g.standard_normal((8192, 4096)).astype(np.float32)
    y = hip.softmax(hip.tensor(x))
    yn = y.numpy()
    t_dy = hip.tensor(dy)
    got = hip.softmax_backward(y, t_dy).numpy()
    softmax_bw_check(got, yn, dy, "softmax backward 8192x4096")
    assert np.array_equal(got, hip.softmax_backward(y, t_dy).numpy())


# ---- matmul backward -------------------------------------------------------

def mm_check(got, want, what):
    atol = 1e-4 * float(np.abs(want).max() or 1.0)
    assert_close(got, want, 2e-3, atol, what)


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (5, 7, 3), (64, 784, 128), (64, 128, 10),
                                   (130, 17, 129), (257, 64, 255), (32, 4096, 96)])
def test_matmul_backward_shapes(hip, m, k, n):
    g = rng(m * 3 + k * 5 + n)
    a = g.normal(0, 1 / np.sqrt(k), (m, k)).astype(np.float32)
    b = g.normal(0, 1, (k, n)).astype(np.float32)
    dc = g.normal(0, 1, (m, n)).astype(np.float32)
    da, db = hip.matmul_backward(hip.tensor(a), hip.tensor(b), hip.tensor(dc))
    wa, wb = oracle.matmul_backward(a, b, dc)
    assert da.shape == (m, k) and db.shape == (k, n)
    mm_check(da.numpy(), wa, f"dA {m}x{k}x{n}")
    mm_check(db.numpy(), wb, f"dB {m}x{k}x{n}")


def test_matmul_backward_leading_dims_and_skips(hip):
    g = rng(9)
    a = g.standard_normal((2, 3, 5)).astype(np.float32)
    b = g.standard_normal((5, 4)).astype(np.float32)
    dc = g.standard_normal((2, 3, 4)).astype(np.float32)
    ta, tb, tdc = hip.tensor(a), hip.tensor(b), hip.tensor(dc)
    da, db = hip.matmul_backward(ta, tb, tdc)
    wa, wb = oracle.matmul_backward(a, b, dc)
    assert da.shape == (2, 3, 5)
    mm_check(da.numpy(), wa, "dA leading dims")
    mm_check(db.numpy(), wb, "dB leading dims")
    only_a, none_b = hip.matmul_backward(ta, tb, tdc, want_b=False)
    assert none_b is None and np.array_equal(only_a.numpy(), da.numpy())
    with pytest.raises(hip.CloveError):
        hip.matmul_backward(ta, tb, hip.tensor(np.ones((6, 5), np.float32)))


def test_matmul_backward_4096(hip):
    """Config-4 size: every 97th row of dA and dB against float64 numpy."""
    g = rng(3)
    K = 4096
    a = g.normal(0, 1 / 64, (K, K)).astype(np.float32)
    b = g.normal(0, 1 / 64, (K, K)).astype(np.float32)
    dc = g.normal(0, 1, (K, K)).astype(np.float32)
    da, db = hip.matmul_backward(hip.tensor(a), hip.tensor(b), hip.tensor(dc))
    da, db = da.numpy(), db.numpy()
    sub = slice(0, K, 97)
    ra = dc[sub].astype(np.float64) @ b.astype(np.float64).T
    rb = a.astype(np.float64).T[sub] @ dc.astype(np.float64)
    assert np.max(np.abs(da[sub] - ra)) < 2e-3 * np.abs(ra).max()
    assert np.max(np.abs(db[sub] - rb)) < 2e-3 * np.abs(rb).max()


@pytest.mark.parametrize("m,k,n", [(4096, 4096, 4096), (4096, 1024, 2048), (2048, 4096, 4096),
                                   (2048, 2048, 2048), (2048, 2048, 1024),
                                   (3, 5, 7), (1000, 300, 500),
                                   # ragged tiles and K tails (edge form of the DMA kernel)
                                   (4100, 4096, 4100), (4100, 2052, 2052), (2052, 4100, 4104),
                                   # 64x128 tiles: unsplit, split, ragged with a K tail
                                   (768, 4096, 4096), (1536, 1536, 1536), (3000, 3000, 3000),
                                   (2100, 2100, 2100)])
def test_matmul_backward_transposed_loads_match_copies(hip, monkeypatch, m, k, n):
    """Where the plan allows, the backward's GEMMs read b^T / a^T straight
    from b / a, by buffer->LDS DMA (the default; ragged tiles and K tails
    included) or through registers (CLOVE_GEMM_DMA=0, interior tiles); the
    result must be the same bits as transposing first
    (CLOVE_GEMM_TRANSPOSED=0), and shapes the direct path does not take must
    give the same bits either way too."""
    g = rng(m + 3 * k + 7 * n)
    a = g.normal(0, 1 / np.sqrt(k), (m, k)).astype(np.float32)
    b = g.normal(0, 1 / np.sqrt(k), (k, n)).astype(np.float32)
    dc = g.normal(0, 1, (m, n)).astype(np.float32)
    ta, tb, tdc = hip.tensor(a), hip.tensor(b), hip.tensor(dc)
    da, db = (t.numpy() for t in hip.matmul_backward(ta, tb, tdc))
    monkeypatch.setenv("CLOVE_GEMM_DMA", "0")
    da1, db1 = (t.numpy() for t in hip.matmul_backward(ta, tb, tdc))
    assert np.array_equal(da, da1) and np.array_equal(db, db1)
    monkeypatch.delenv("CLOVE_GEMM_DMA")
    monkeypatch.setenv("CLOVE_GEMM_TRANSPOSED", "0")
    da0, db0 = (t.numpy() for t in hip.matmul_backward(ta, tb, tdc))
    assert np.array_equal(da, da0) and np.array_equal(db, db0)


# ---- broadcast operand gradient (add / sub backward) -----------------------

@pytest.mark.parametrize("n,nb", [(4096 * 4096, 4096), (1000, 7), (999, 10), (12, 1),
                                  (1 << 24, 1), (5, 8), (64 * 300 + 5, 64), (63 * 1000, 63),
                                  (65 * 777, 65), (784 * 128, 128), (640, 10), (0, 3),
                                  # a partial block of column quads and a partial last row;
                                  # more than 16384 x 64 rows (chunks of more than 64 rows)
                                  (4100 * 70 + 13, 4100), (530000 * 64 + 3, 64),
                                  (1100000 * 64 + 3, 64),
                                  # the one-pass strip kernel (nb >= 16 per CU): fewer rows
                                  # than a workgroup's row groups, a partial last row, wide b
                                  (4096 * 3, 4096), (8192 * 33 + 100, 8192), (16384 * 300, 16384)])
def test_broadcast_grad_exact(hip, n, nb):
    g = rng(n % 1000 + nb)
    go = g.integers(-8, 9, n).astype(np.float32)
    tg = hip.tensor(go) if n else hip.empty((0,))
    for negate in (False, True):
        got = hip.broadcast_grad(tg, nb, negate).numpy()
        assert np.array_equal(got, oracle.bias_grad(go, nb, negate)), (n, nb, negate)


def test_broadcast_grad_float_data(hip):
    g = rng(50)
    go = g.standard_normal((512, 4096)).astype(np.float32)
    tg = hip.tensor(go)
    got = hip.broadcast_grad(tg, 4096).numpy()
    want = oracle.bias_grad(go, 4096)
    scale = np.sqrt(512) * 1e-5  # error of a sum of 512 unit normals in another order
    assert np.all(np.abs(got - want) <= 1e-4 * np.abs(want) + scale)
    assert np.array_equal(got, hip.broadcast_grad(tg, 4096).numpy())
    with pytest.raises(hip.CloveError):
        hip.broadcast_grad(tg, 0)


# ---- losses ----------------------------------------------------------------

@pytest.mark.parametrize("rows,cols", [(37, 23), (64, 10), (8, 4096), (3, 8200), (1, 1)])
def test_cross_entropy(hip, rows, cols):
    g = rng(rows + cols)
    logits = g.normal(0, 3, (rows, cols)).astype(np.float32)
    t = g.integers(0, cols, rows).astype(np.float32)
    tl, tt = hip.tensor(logits), hip.tensor(t)
    loss = hip.cross_entropy(tl, tt).numpy()
    want = oracle.cross_entropy(logits, t)
    assert loss.shape == (1, 1)
    assert abs(loss[0, 0] - want[0, 0]) <= 1e-4 * abs(want[0, 0]) + 1e-7
    gl = hip.tensor(np.array([1.5], np.float32))
    grad = hip.cross_entropy_backward(tl, tt, gl).numpy()
    wg = oracle.cross_entropy_backward(logits, t, 1.5)
    assert_close(grad, wg, 1e-4, 1e-4 * 1.5 / rows * 1e-2, f"ce backward {rows}x{cols}")


@pytest.mark.parametrize("cols", [1028, 2052, 4100, 8196, 12000, 32768, 32772])
def test_wide_rows_backward_and_losses(hip, cols):
    """Widths that take the one-workgroup-per-row kernels (every vectors-per-
    thread variant) and one past them.  The targets sit in the row's first
    and last columns and in every thread slot, so l[target] is fetched from
    each position it can occupy."""
    g = rng(cols + 3)
    slots = [4 * 512 * k + 5 for k in range(16) if 4 * 512 * k + 5 < cols]
    t = np.array([0, cols - 1] + slots, np.float32)
    rows = len(t)
    logits = g.normal(0, 3, (rows, cols)).astype(np.float32)
    tl, tt = hip.tensor(logits), hip.tensor(t)
    loss = hip.cross_entropy(tl, tt).numpy()[0, 0]
    want = oracle.cross_entropy(logits, t)[0, 0]
    assert abs(loss - want) <= 1e-4 * abs(want) + 1e-7, (loss, want)
    gl = hip.tensor(np.array([1.5], np.float32))
    grad = hip.cross_entropy_backward(tl, tt, gl).numpy()
    wg = oracle.cross_entropy_backward(logits, t, 1.5)
    assert_close(grad, wg, 1e-4, 1e-4 * 1.5 / rows * 1e-2, f"ce backward {rows}x{cols}")
    y = oracle.softmax(g.normal(0, 2, (3, cols)).astype(np.float32))
    dy = g.standard_normal((3, cols)).astype(np.float32)
    got = hip.softmax_backward(hip.tensor(y), hip.tensor(dy)).numpy()
    softmax_bw_check(got, y, dy, f"softmax backward 3x{cols}")


def test_cross_entropy_config3_full(hip):
    g = rng(2)
    logits = g.normal(0, 2, (8192, 4096)).astype(np.float32)
    t = g.integers(0, 4096, 8192).astype(np.float32)
    tl, tt = hip.tensor(logits), hip.tensor(t)
    loss = hip.cross_entropy(tl, tt).numpy()[0, 0]
    want = oracle.cross_entropy(logits, t)[0, 0]
    assert abs(loss - want) <= 1e-4 * abs(want)
    assert loss == hip.cross_entropy(tl, tt).numpy()[0, 0]
    grad = hip.cross_entropy_backward(tl, tt, hip.tensor(np.ones(1, np.float32))).numpy()
    wg = oracle.cross_entropy_backward(logits, t, 1.0)
    assert_close(grad, wg, 1e-4, 1e-10, "ce backward 8192x4096")


def test_cross_entropy_targets_edge_cases(hip):
    g = rng(51)
    logits = g.standard_normal((6, 5)).astype(np.float32)
    tl = hip.tensor(logits)
    # fewer targets than rows: only those rows count, divided by all rows
    t3 = np.array([0, 4, 2], np.float32)
    got = hip.cross_entropy(tl, hip.tensor(t3)).numpy()[0, 0]
    assert abs(got - oracle.cross_entropy(logits, t3)[0, 0]) <= 1e-5
    grad = hip.cross_entropy_backward(tl, hip.tensor(t3), hip.tensor(np.ones(1, np.float32)))
    assert np.all(grad.numpy()[3:] == 0)
    # negative / NaN targets read class 0 (Rust's saturating `as usize`)
    tn = np.array([-2, np.nan, 0, 0, 0, 0], np.float32)
    a = hip.cross_entropy(tl, hip.tensor(tn)).numpy()[0, 0]
    b = hip.cross_entropy(tl, hip.tensor(np.zeros(6, np.float32))).numpy()[0, 0]
    assert a == b
    # a class >= cols is reported at the next synchronising call
    hip.cross_entropy(tl, hip.tensor(np.array([0, 5], np.float32)))
    with pytest.raises(hip.CloveError) as e:
        hip.synchronize()
    assert e.value.code == 7  # CLOVE_HIP_ERR_RANGE
    hip.synchronize()  # the flag is cleared once reported


@pytest.mark.parametrize("shape", [(1,), (33, 17), (4096, 4096), (7, 1000)])
def test_mse(hip, shape):
    """Against float64 at every size, and against the oracle where its
    sequential f32 fold is itself accurate: at 16.7M terms of ~2 the running
    sum's ulp reaches 2 and the reference's fold ends ~3% low (1.944 for a
    true 2.000); the GPU's tree sum stays within 1e-4 of float64."""
    g = rng(sum(shape))
    p = g.standard_normal(shape).astype(np.float32)
    t = g.standard_normal(shape).astype(np.float32)
    tp, tt = hip.tensor(p), hip.tensor(t)
    loss = hip.mse(tp, tt).numpy()[0, 0]
    exact = np.mean((p.astype(np.float64) - t) ** 2)
    assert abs(loss - exact) <= 1e-4 * exact
    if p.size <= 1 << 20:
        want = oracle.mse(p, t)[0, 0]
        assert abs(loss - want) <= 1e-4 * abs(want)
    assert loss == hip.mse(tp, tt).numpy()[0, 0]
    grad = hip.mse_backward(tp, tt, hip.tensor(np.array([0.25], np.float32))).numpy()
    assert_close(grad, oracle.mse_backward(p, t, 0.25), 1e-6, 1e-30, "mse backward")


def test_mse_edge_cases(hip):
    z = hip.empty((0,))
    assert np.isnan(hip.mse(z, z).numpy()[0, 0])  # 0 / 0, as the reference computes
    with pytest.raises(hip.CloveError):
        hip.mse(hip.tensor(np.ones(4, np.float32)), hip.tensor(np.ones(3, np.float32)))


def test_cross_entropy_row_pairs_edge_cases(hip):
    """The two-rows-per-workgroup forward (widths 1025-4096): fewer targets
    than rows (a pair with one counted row), an odd row count, and a class
    >= cols in the second row of a pair (reported; that row counts 0)."""
    g = rng(52)
    for cols in (1028, 2048, 4096):
        logits = g.normal(0, 3, (9, cols)).astype(np.float32)
        tl = hip.tensor(logits)
        t5 = g.integers(0, cols, 5).astype(np.float32)
        got = hip.cross_entropy(tl, hip.tensor(t5)).numpy()[0, 0]
        want = oracle.cross_entropy(logits, t5)[0, 0]
        assert abs(got - want) <= 1e-4 * abs(want) + 1e-7, (cols, got, want)
        bad = t5.copy()
        bad[3] = cols
        got = hip.cross_entropy(tl, hip.tensor(bad))
        with pytest.raises(hip.CloveError) as e:
            hip.synchronize()
        assert e.value.code == 7
        keep = np.array([0, 1, 2, 4], np.int64)  # the rows that still count
        # the loss over the kept rows, times their count, over all 9 rows
        want = oracle.cross_entropy(logits[keep], t5[keep])[0, 0] * 4 / 9
        assert abs(got.numpy()[0, 0] - want) <= 1e-4 * abs(want) + 1e-7
