"""Pins of the CPU oracle (CPU only).

The oracle restates Clove's Rayon kernels; these tests pin it against
(1) Clove's own known-answer tests (tests/golden/clove_kats.json),
(2) independent float64 library implementations (numpy, torch, scipy),
(3) closed forms and invariants chosen so that a plausible mistake -- a
wrong broadcast index, a transposed operand, an unbiased variance, eps
outside the square root, a fused multiply-add, a pairwise instead of a
sequential sum, a wrong block-table index -- fails at least one of them.
"""
import json
import os

import numpy as np
import pytest

import oracle
from conftest import assert_close, rng

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "clove_kats.json")


@pytest.fixture(scope="module")
def kats():
    with open(GOLDEN) as f:
        return json.load(f)


# ---------------------------------------------------------------------------
# Clove's own known answers
# ---------------------------------------------------------------------------

def test_kat_sub_mul(kats):
    for name, fn in (("sub", oracle.sub), ("mul", oracle.mul)):
        k = kats[name]
        out = fn(np.array(k["a"], np.float32), np.array(k["b"], np.float32))
        assert np.array_equal(out, np.array(k["out"], np.float32)), name


def test_kat_trig(kats):
    for name, fn in (("sin", oracle.sin), ("cos", oracle.cos)):
        k = kats[name]
        out = fn(np.array(k["x"], np.float32))
        assert np.all(np.abs(out - np.array(k["out"])) < k["tol"]), name


def test_kat_linear_relu(kats):
    k = kats["linear_relu"]
    x, w, b = (np.array(k[n], np.float32) for n in ("x", "w", "b"))
    out = oracle.relu(oracle.add(oracle.matmul(x, w), b))
    assert np.all(np.abs(out - np.array(k["out"])) < k["tol"])


# ---------------------------------------------------------------------------
# elementwise
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("nb", [1, 3, 4, 7, 12, 64])
def test_binary_broadcast_matches_numpy(nb):
    g = rng(10 + nb)
    a = g.standard_normal((8, 96), dtype=np.float32)
    b = g.standard_normal(nb, dtype=np.float32)
    bb = np.resize(b, a.size).reshape(a.shape)  # b[i % nb], built independently
    assert np.array_equal(oracle.add(a, b), a + bb)
    assert np.array_equal(oracle.sub(a, b), a - bb)
    assert np.array_equal(oracle.mul(a, b), a * bb)


def test_mul_scalar_and_relu_exact():
    g = rng(11)
    a = g.standard_normal(1000, dtype=np.float32)
    a[:4] = [0.0, -0.0, np.inf, -np.inf]
    assert np.array_equal(oracle.mul_scalar(a, 0.37), a * np.float32(0.37))
    r = oracle.relu(a)
    assert np.array_equal(r, np.where(a > 0, a, np.float32(0)))
    assert not np.signbit(r[1])  # relu(-0.0) is +0.0 (the `else { 0.0 }` arm)
    assert np.isnan(oracle.relu(np.array([np.nan], np.float32)))[0] == False  # NaN > 0 is false


def test_gelu_against_torch_float64():
    torch = pytest.importorskip("torch")
    g = rng(12)
    x = np.concatenate([g.standard_normal(20000, dtype=np.float32) * 3,
                        np.linspace(-10, 10, 2001, dtype=np.float32)])
    want = torch.nn.functional.gelu(torch.from_numpy(x.astype(np.float64)),
                                    approximate="tanh").numpy()
    assert_close(oracle.gelu(x), want, rtol=2e-6, atol=2e-7, what="gelu")
    assert oracle.gelu(np.zeros(1, np.float32))[0] == 0.0


def test_gelu_uses_f32_sqrt_2_over_pi():
    # (2/pi).sqrt() in f32 is 0x3F4C4229; the WGSL literal 0.7978845608 is one
    # ulp higher.  Evaluate both step by step in numpy f32 (IEEE, no FMA) and
    # check the oracle matches the f32 constant on inputs where they differ.
    x = np.linspace(0.5, 3.0, 4001, dtype=np.float32)
    f = np.float32
    def step(k):
        x3 = (x * x) * x
        inner = k * (x + f(0.044715) * x3)
        return f(0.5) * x * (f(1) + np.tanh(inner.astype(np.float64)).astype(np.float32))
    k_cpu = np.sqrt(f(2) / f(np.pi))
    assert k_cpu.view(np.uint32) == 0x3F4C4229
    ref = step(k_cpu)
    alt = step(f(0.7978845608))
    differ = ref != alt
    assert differ.sum() > 10
    got = oracle.gelu(x)
    # tanhf in glibc and numpy's f64->f32 tanh may differ by an ulp; the
    # constant choice shows up in the majority vote on the differing inputs.
    assert (got[differ] == ref[differ]).mean() > (got[differ] == alt[differ]).mean()


def test_sigmoid_tanh_trig_against_float64():
    g = rng(13)
    x = g.standard_normal(50000, dtype=np.float32) * 4
    xd = x.astype(np.float64)
    assert_close(oracle.sigmoid(x), 1 / (1 + np.exp(-xd)), rtol=3e-7, atol=1e-30, what="sigmoid")
    assert_close(oracle.tanh(x), np.tanh(xd), rtol=3e-7, atol=1e-30, what="tanh")
    assert_close(oracle.sin(x), np.sin(xd), rtol=0, atol=2e-7, what="sin")
    assert_close(oracle.cos(x), np.cos(xd), rtol=0, atol=2e-7, what="cos")


# ---------------------------------------------------------------------------
# softmax / layer norm
# ---------------------------------------------------------------------------

def test_softmax_against_torch_float64():
    torch = pytest.importorskip("torch")
    g = rng(14)
    x = g.normal(0, 2, (64, 513)).astype(np.float32)
    want = torch.softmax(torch.from_numpy(x.astype(np.float64)), dim=-1).numpy()
    assert_close(oracle.softmax(x), want, rtol=1e-5, atol=1e-12, what="softmax")


def test_softmax_closed_forms():
    c = oracle.softmax(np.full((2, 4096), 3.25, np.float32))
    assert np.all(c == np.float32(1 / 4096))          # constant row: exactly 1/n
    oh = oracle.softmax(np.array([[0.0, 0.0, 120.0, 0.0]], np.float32))
    # one-hot on a large gap: exp(-120) underflows to 0 in f32
    assert oh[0, 2] == 1.0 and np.all(oh[0, [0, 1, 3]] == 0.0)
    g = rng(15)
    x = g.normal(0, 2, (16, 1000)).astype(np.float32)
    s = oracle.softmax(x).astype(np.float64).sum(-1)
    assert np.all(np.abs(s - 1) < 1000 * 6e-8)         # rows sum to 1 within n*u


def test_layer_norm_against_torch_float64():
    torch = pytest.importorskip("torch")
    g = rng(16)
    for cols, scale in ((8, 1.0), (4096, 2.0), (33, 1e-3)):
        x = (g.standard_normal((32, cols)) * scale).astype(np.float32)
        gamma = g.uniform(0.5, 1.5, cols).astype(np.float32)
        beta = g.uniform(-0.1, 0.1, cols).astype(np.float32)
        want = torch.nn.functional.layer_norm(
            torch.from_numpy(x.astype(np.float64)), (cols,),
            torch.from_numpy(gamma.astype(np.float64)), torch.from_numpy(beta.astype(np.float64)),
            eps=1e-5).numpy()
        # cols=8 separates biased from unbiased variance (a 6% difference);
        # scale=1e-3 makes var ~ eps, which separates eps inside / outside sqrt.
        assert_close(oracle.layer_norm(x, gamma, beta), want, rtol=1e-4, atol=1e-5,
                     what=f"layer_norm cols={cols}")


def test_layer_norm_constant_row_is_beta():
    beta = np.linspace(-1, 1, 64, dtype=np.float32)
    out = oracle.layer_norm(np.full((3, 64), 7.5, np.float32), np.full(64, 2.0, np.float32), beta)
    assert np.array_equal(out, np.broadcast_to(beta, out.shape))


# ---------------------------------------------------------------------------
# matmul
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (3, 5, 7), (17, 64, 9), (64, 784, 128)])
def test_matmul_against_numpy_float64(m, k, n):
    g = rng(17 + m)
    a = g.standard_normal((m, k)).astype(np.float32)
    b = g.standard_normal((k, n)).astype(np.float32)
    want = a.astype(np.float64) @ b.astype(np.float64)
    scale = np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)
    err = np.abs(oracle.matmul(a, b) - want)
    assert np.all(err <= k * 6e-8 * scale + 1e-30)


def test_matmul_identity_permutation_rank1():
    g = rng(18)
    a = g.standard_normal((6, 9)).astype(np.float32)
    assert np.array_equal(oracle.matmul(a, np.eye(9, dtype=np.float32)), a)
    p = np.eye(9, dtype=np.float32)[g.permutation(9)]
    assert np.array_equal(oracle.matmul(a, p), a @ p)  # column permutation, exact
    u = g.standard_normal((5, 1)).astype(np.float32)
    v = g.standard_normal((1, 4)).astype(np.float32)
    assert np.array_equal(oracle.matmul(u, v), u * v)  # rank 1, k = 1: exact products


def test_matmul_leading_dims():
    g = rng(19)
    a = g.standard_normal((2, 3, 5)).astype(np.float32)
    b = g.standard_normal((5, 4)).astype(np.float32)
    out = oracle.matmul(a, b)
    assert out.shape == (2, 3, 4)
    assert np.array_equal(out.reshape(6, 4), oracle.matmul(a.reshape(6, 5), b))


def test_matmul_is_a_sequential_f32_fold_without_fma():
    # Sequential f32: (1e8 + 1) rounds to 1e8, then - 1e8 gives 0; a pairwise
    # or f64 sum gives 1.
    a = np.array([[1e8, 1.0, -1e8]], np.float32)
    b = np.ones((3, 1), np.float32)
    assert oracle.matmul(a, b)[0, 0] == 0.0
    # Separate roundings: a*b rounds before the add.  Emulate one dot product
    # step by step with numpy f32 scalars (IEEE, never contracted).
    g = rng(20)
    x = g.standard_normal((1, 257)).astype(np.float32)
    y = g.standard_normal((257, 1)).astype(np.float32)
    s = np.float32(0)
    for p in range(257):
        s = np.float32(s + np.float32(x[0, p] * y[p, 0]))
    assert oracle.matmul(x, y)[0, 0] == s


# ---------------------------------------------------------------------------
# paged attention
# ---------------------------------------------------------------------------

def make_paged(seed, B=3, H=2, D=64, bs=16, nb=40, max_blocks=6, ctx=None):
    g = rng(seed)
    kv = g.standard_normal((2, nb, bs, H, D)).astype(np.float32)
    q = g.standard_normal((B, H, D)).astype(np.float32)
    kn = g.standard_normal((B, H, D)).astype(np.float32)
    vn = g.standard_normal((B, H, D)).astype(np.float32)
    bt = g.permutation(nb)[: B * max_blocks].reshape(B, max_blocks).astype(np.int32)
    if ctx is None:
        ctx = g.integers(1, max_blocks * bs + 1, B)
    cl = np.asarray(ctx, np.int32)
    return q, kn, vn, kv, bt, cl


def gather_reference(q, kn, vn, kv, bt, cl, scale):
    """Contiguous K/V by explicit slot arithmetic, then torch SDPA in f64."""
    torch = pytest.importorskip("torch")
    _, nb, bs, H, D = kv.shape
    out = np.zeros(q.shape, np.float64)
    for b in range(cl.size):
        ctx = int(cl[b])
        if ctx == 0:
            continue
        slots = [int(bt[b, t // bs]) * bs + t % bs for t in range(ctx)]
        K = kv[0].reshape(nb * bs, H, D)[slots].astype(np.float64)
        V = kv[1].reshape(nb * bs, H, D)[slots].astype(np.float64)
        if kn is not None:
            K[-1], V[-1] = kn[b], vn[b]
        qq = torch.from_numpy(q[b].astype(np.float64))[:, None, :]          # [H, 1, D]
        KK = torch.from_numpy(np.ascontiguousarray(K.transpose(1, 0, 2)))   # [H, ctx, D]
        VV = torch.from_numpy(np.ascontiguousarray(V.transpose(1, 0, 2)))
        o = torch.nn.functional.scaled_dot_product_attention(qq, KK, VV, scale=float(scale))
        out[b] = o[:, 0, :].numpy()
    return out


@pytest.mark.parametrize("with_new", [False, True])
def test_paged_against_torch_sdpa(with_new):
    q, kn, vn, kv, bt, cl = make_paged(21, ctx=[1, 37, 96])
    if not with_new:
        kn = vn = None
    scale = 1 / np.sqrt(np.float32(64))
    want = gather_reference(q, kn, vn, kv, bt, cl, scale)
    assert_close(oracle.paged_attention(q, kn, vn, kv, bt, cl), want, 1e-5, 1e-6, "f32 oracle")
    assert_close(oracle.paged_attention(q, kn, vn, kv, bt, cl, f64=True), want, 1e-12, 1e-14,
                 "f64 oracle")


def test_paged_invariants():
    q, kn, vn, kv, bt, cl = make_paged(22, ctx=[1, 50, 80])
    B, H, D = q.shape
    # ctx = 1: the output is V of the single token.
    out = oracle.paged_attention(q, None, None, kv, bt, cl)
    slot0 = int(bt[0, 0]) * 16
    assert np.array_equal(out[0], kv[1].reshape(-1, H, D)[slot0])
    # q = 0: uniform weights, the output is the mean of V over the context.
    out0 = oracle.paged_attention(np.zeros_like(q), None, None, kv, bt, cl, f64=True)
    slots = [int(bt[1, t // 16]) * 16 + t % 16 for t in range(50)]
    assert_close(out0[1], kv[1].reshape(-1, H, D)[slots].astype(np.float64).mean(0), 1e-12, 1e-14)
    # V constant per head: the output is that constant, whatever the scores.
    kv2 = kv.copy()
    kv2[1] = np.arange(H, dtype=np.float32)[None, None, :, None] + 0.5
    o2 = oracle.paged_attention(q, None, None, kv2, bt, cl)
    assert_close(o2, np.broadcast_to((np.arange(H) + 0.5)[None, :, None], o2.shape), 1e-6, 0)


def test_paged_new_token_equals_cache_write():
    q, kn, vn, kv, bt, cl = make_paged(23, ctx=[5, 16, 17])
    with_new = oracle.paged_attention(q, kn, vn, kv, bt, cl)
    kv2 = kv.copy()
    for b in range(3):
        t = int(cl[b]) - 1
        kv2[0, bt[b, t // 16], t % 16] = kn[b]
        kv2[1, bt[b, t // 16], t % 16] = vn[b]
    assert np.array_equal(with_new, oracle.paged_attention(q, None, None, kv2, bt, cl))


def test_paged_permuted_pool_equals_contiguous():
    # The same logical cache stored contiguously (identity table) and
    # scattered through a permuted table gives bit-identical outputs.
    q, kn, vn, kv, bt, cl = make_paged(24, ctx=[70, 3, 96])
    out = oracle.paged_attention(q, None, None, kv, bt, cl)
    B, mb = bt.shape
    contig = np.zeros((2, B * mb) + kv.shape[2:], np.float32)
    for b in range(B):
        for j in range(mb):
            contig[:, b * mb + j] = kv[:, bt[b, j]]
    ident = np.arange(B * mb, dtype=np.int32).reshape(B, mb)
    assert np.array_equal(out, oracle.paged_attention(q, None, None, contig, ident, cl))


def test_paged_slots_brute_force():
    g = rng(25)
    bt = g.permutation(100)[:40].reshape(5, 8).astype(np.int32)
    cl = np.array([0, 1, 16, 17, 128], np.int32)
    got = oracle.paged_slots(bt, cl, 16, 130)
    for b in range(5):
        for t in range(130):
            want = bt[b, t // 16] * 16 + t % 16 if t < cl[b] else -1
            assert got[b, t] == want


def test_paged_empty_context_is_zero():
    q, kn, vn, kv, bt, cl = make_paged(26, ctx=[0, 5, 0])
    out = oracle.paged_attention(q, None, None, kv, bt, cl)
    assert np.all(out[0] == 0) and np.all(out[2] == 0) and np.any(out[1] != 0)


# ---------------------------------------------------------------------------
# compositions
# ---------------------------------------------------------------------------

def test_chain_against_float64_composition():
    torch = pytest.importorskip("torch")
    g = rng(27)
    a, b, c, d = (g.standard_normal(4096).astype(np.float32) for _ in range(4))
    ops = [("mul", -1, -2), ("add", 0, -3), ("gelu", 1), ("mul", 2, -4)]
    (out,) = oracle.chain(ops, [a, b, c, d])
    x = torch.from_numpy(a.astype(np.float64) * b + c)
    want = torch.nn.functional.gelu(x, approximate="tanh").numpy() * d
    assert_close(out, want, 1e-5, 1e-6, "gelu(a*b+c)*d")


def test_mlp_forward_against_float64():
    g = rng(28)
    x = g.random((8, 20)).astype(np.float32)
    w1 = g.uniform(-0.5, 0.5, (20, 16)).astype(np.float32)
    b1 = g.uniform(-1, 1, (1, 16)).astype(np.float32)
    w2 = g.uniform(-0.5, 0.5, (16, 10)).astype(np.float32)
    b2 = g.uniform(-1, 1, (1, 10)).astype(np.float32)
    h = np.maximum(x.astype(np.float64) @ w1 + b1, 0)
    z = h @ w2 + b2
    want = np.exp(z - z.max(1, keepdims=True))
    want /= want.sum(1, keepdims=True)
    assert_close(oracle.mlp_forward(x, w1, b1, w2, b2), want, 1e-5, 1e-9, "mlp")


def test_paged_kv_append_is_the_cache_write():
    q, kn, vn, kv, bt, cl = make_paged(29, ctx=[0, 16, 33])
    kv2 = oracle.paged_kv_append(kv, kn, vn, bt, cl)
    # only slot ctx-1 of sequences 1 and 2 changed, in both planes
    changed = np.argwhere(np.any(kv2 != kv, axis=(3, 4)))
    want = sorted([(p, int(bt[b, (cl[b] - 1) // 16]), int((cl[b] - 1) % 16))
                   for p in (0, 1) for b in (1, 2)])
    assert sorted(map(tuple, changed.tolist())) == want
    assert np.array_equal(oracle.paged_attention(q, None, None, kv2, bt, cl)[1:],
                          oracle.paged_attention(q, kn, vn, kv, bt, cl)[1:])


# ---------------------------------------------------------------------------
# backward passes and losses
# ---------------------------------------------------------------------------

def _torch():
    return pytest.importorskip("torch")


def test_relu_backward_exact():
    g = rng(40)
    x = g.standard_normal(5000).astype(np.float32)
    x[:3] = [0.0, -0.0, np.nan]
    go = g.standard_normal(5000).astype(np.float32)
    got = oracle.relu_backward(x, go)
    assert np.array_equal(got, np.where(x > 0, go, np.float32(0)))
    # relu's output gives the same mask as its input
    assert np.array_equal(oracle.relu_backward(oracle.relu(x), go), got)


def test_gelu_backward_against_torch_autograd():
    torch = _torch()
    g = rng(41)
    x = np.concatenate([g.standard_normal(20000).astype(np.float32) * 3,
                        np.linspace(-8, 8, 1601, dtype=np.float32)])
    go = g.standard_normal(x.size).astype(np.float32)
    xt = torch.from_numpy(x.astype(np.float64)).requires_grad_()
    torch.nn.functional.gelu(xt, approximate="tanh").backward(torch.from_numpy(go.astype(np.float64)))
    # The reference's f32 formula loses absolute (not relative) accuracy where
    # its terms cancel: near the derivative's zero (x ~ -0.75), and at |x| ~ 8
    # where 1 + tanh cancels and 1 - t^2 (~6e-8 absolute error) is scaled by
    # x*c*(1 + 0.134x^2) ~ 30.  So the error bound is relative to the result
    # plus absolute in the derivative, times |grad_out|.
    got, want = oracle.gelu_backward(x, go), xt.grad.numpy()
    d_abs = np.where(np.abs(x) < 3, 2e-7, 3e-6)
    assert np.all(np.abs(got - want) <= 3e-6 * np.abs(want) + d_abs * np.abs(go) + 1e-30)
    # the derivative at 0 is exactly 1/2
    assert oracle.gelu_backward(np.zeros(1, np.float32), np.ones(1, np.float32))[0] == 0.5


def test_gelu_backward_against_central_difference():
    # independent of torch: (gelu(x+h) - gelu(x-h)) / 2h in float64
    x = np.linspace(-6, 6, 241).astype(np.float64)
    c = np.sqrt(2 / np.pi)
    gelu = lambda v: 0.5 * v * (1 + np.tanh(c * (v + 0.044715 * v ** 3)))
    h = 1e-5
    fd = (gelu(x + h) - gelu(x - h)) / (2 * h)
    got = oracle.gelu_backward(x.astype(np.float32), np.ones_like(x, dtype=np.float32))
    assert_close(got, fd, rtol=1e-5, atol=1e-6, what="gelu backward vs finite difference")


def test_softmax_backward_against_torch_autograd():
    torch = _torch()
    g = rng(42)
    x = g.normal(0, 2, (48, 257)).astype(np.float32)
    dy = g.standard_normal((48, 257)).astype(np.float32)
    xt = torch.from_numpy(x.astype(np.float64)).requires_grad_()
    torch.softmax(xt, dim=-1).backward(torch.from_numpy(dy.astype(np.float64)))
    y = oracle.softmax(x)
    assert_close(oracle.softmax_backward(y, dy), xt.grad.numpy(), rtol=1e-4, atol=1e-7,
                 what="softmax backward")


def test_softmax_backward_closed_forms():
    g = rng(43)
    y = oracle.softmax(g.standard_normal((16, 100)).astype(np.float32))
    # a constant upstream gradient has no effect on softmax: dx = 0
    dx = oracle.softmax_backward(y, np.full_like(y, 3.0))
    assert np.abs(dx).max() < 1e-6
    # rows of dx always sum to 0 (sum_j y_j (g_j - s) = s - s)
    dx = oracle.softmax_backward(y, g.standard_normal(y.shape).astype(np.float32))
    assert np.abs(dx.sum(axis=1)).max() < 1e-5


@pytest.mark.parametrize("m,k,n", [(5, 7, 3), (17, 33, 9), (64, 128, 10)])
def test_matmul_backward_against_numpy_float64(m, k, n):
    g = rng(m + k + n)
    a = g.standard_normal((m, k)).astype(np.float32)
    b = g.standard_normal((k, n)).astype(np.float32)
    dc = g.standard_normal((m, n)).astype(np.float32)
    da, db = oracle.matmul_backward(a, b, dc)
    ad, bd, cd = (v.astype(np.float64) for v in (a, b, dc))
    # non-square shapes: a transposed operand would not even have the shape
    assert da.shape == (m, k) and db.shape == (k, n)
    u = np.finfo(np.float32).eps
    assert np.all(np.abs(da - cd @ bd.T) <= n * u * (np.abs(cd) @ np.abs(bd).T) + 1e-30)
    assert np.all(np.abs(db - ad.T @ cd) <= m * u * (np.abs(ad).T @ np.abs(cd)) + 1e-30)


def test_matmul_backward_against_torch_autograd():
    torch = _torch()
    g = rng(44)
    a = g.standard_normal((2, 6, 11)).astype(np.float32)
    b = g.standard_normal((11, 4)).astype(np.float32)
    dc = g.standard_normal((2, 6, 4)).astype(np.float32)
    at = torch.from_numpy(a.astype(np.float64)).requires_grad_()
    bt = torch.from_numpy(b.astype(np.float64)).requires_grad_()
    (at @ bt).backward(torch.from_numpy(dc.astype(np.float64)))
    da, db = oracle.matmul_backward(a, b, dc)
    assert da.shape == a.shape
    assert_close(da, at.grad.numpy(), rtol=1e-5, atol=1e-5, what="dA")
    assert_close(db, bt.grad.numpy(), rtol=1e-5, atol=1e-5, what="dB")


@pytest.mark.parametrize("n,nb", [(4096, 64), (1000, 7), (999, 10), (12, 1), (50, 50)])
def test_bias_grad_against_numpy(n, nb):
    g = rng(n + nb)
    go = g.integers(-8, 9, n).astype(np.float32)  # small integers: every sum is exact
    want = np.zeros(nb, np.float64)
    np.add.at(want, np.arange(n) % nb, go.astype(np.float64))
    assert np.array_equal(oracle.bias_grad(go, nb), want.astype(np.float32))
    assert np.array_equal(oracle.bias_grad(go, nb, negate=True), (-want).astype(np.float32))


def test_bias_grad_is_an_in_order_fold():
    # i % 1 == 0 for all i: (1e8 + 1) + (-1e8) folds to 0 in f32 order
    assert oracle.bias_grad(np.array([1e8, 1.0, -1e8], np.float32), 1)[0] == 0.0


def test_cross_entropy_against_torch_float64():
    torch = _torch()
    g = rng(45)
    logits = g.normal(0, 3, (37, 23)).astype(np.float32)
    t = g.integers(0, 23, 37).astype(np.float32)
    want = torch.nn.functional.cross_entropy(torch.from_numpy(logits.astype(np.float64)),
                                             torch.from_numpy(t.astype(np.int64))).item()
    got = oracle.cross_entropy(logits, t)
    assert got.shape == (1, 1)
    assert abs(got[0, 0] - want) <= 1e-5 * abs(want)
    # uniform logits: the loss is ln(cols) whatever the targets
    assert abs(oracle.cross_entropy(np.zeros((5, 8), np.float32), t[:5] % 8)[0, 0]
               - np.log(8)) < 1e-6


def test_cross_entropy_rows_and_bad_targets():
    g = rng(46)
    logits = g.standard_normal((6, 5)).astype(np.float32)
    t = np.array([0, 4, 2], np.float32)  # only 3 targets: 3 rows count, divided by 6
    full = oracle.cross_entropy(logits[:3], t)[0, 0] * 3 / 6
    assert abs(oracle.cross_entropy(logits, t)[0, 0] - full) < 1e-6
    # negative and NaN targets saturate to class 0 like Rust's `as usize`
    a = oracle.cross_entropy(logits[:2], np.array([-3.0, np.nan], np.float32))
    b = oracle.cross_entropy(logits[:2], np.array([0.0, 0.0], np.float32))
    assert a[0, 0] == b[0, 0]
    with pytest.raises(IndexError):
        oracle.cross_entropy(logits, np.array([5.0], np.float32))


def test_cross_entropy_backward_against_torch_autograd():
    torch = _torch()
    g = rng(47)
    logits = g.normal(0, 2, (19, 31)).astype(np.float32)
    t = g.integers(0, 31, 19).astype(np.float32)
    lt = torch.from_numpy(logits.astype(np.float64)).requires_grad_()
    (torch.nn.functional.cross_entropy(lt, torch.from_numpy(t.astype(np.int64))) * 2.5).backward()
    got = oracle.cross_entropy_backward(logits, t, 2.5)
    assert_close(got, lt.grad.numpy(), rtol=1e-5, atol=1e-8, what="cross entropy backward")
    assert np.abs(got.sum(axis=1)).max() < 1e-6  # softmax minus one-hot sums to 0
    # rows past the targets get no gradient
    part = oracle.cross_entropy_backward(logits, t[:4], 1.0)
    assert np.all(part[4:] == 0) and np.abs(part[:4]).max() > 0


def test_mse_against_numpy_and_torch():
    torch = _torch()
    g = rng(48)
    p = g.standard_normal((33, 17)).astype(np.float32)
    t = g.standard_normal((33, 17)).astype(np.float32)
    want = np.mean((p.astype(np.float64) - t) ** 2)
    assert abs(oracle.mse(p, t)[0, 0] - want) <= 1e-6 * want
    pt = torch.from_numpy(p.astype(np.float64)).requires_grad_()
    (torch.nn.functional.mse_loss(pt, torch.from_numpy(t.astype(np.float64))) * 0.5).backward()
    assert_close(oracle.mse_backward(p, t, 0.5), pt.grad.numpy(), rtol=1e-6, atol=1e-12,
                 what="mse backward")
    assert oracle.mse(p, p)[0, 0] == 0.0


# ---------------------------------------------------------------------------
# AdamW
# ---------------------------------------------------------------------------

def test_adamw_against_torch_float64():
    """Five steps against torch.optim.AdamW in float64 (decoupled decay,
    bias-corrected moments: the same mathematics), fed the unscaled,
    clipped gradients the reference step computes."""
    torch = _torch()
    g = rng(60)
    w0 = g.standard_normal(1000).astype(np.float32)
    grads = [(g.standard_normal(1000) * 65536 * 0.7).astype(np.float32) for _ in range(5)]
    p = torch.nn.Parameter(torch.from_numpy(w0.astype(np.float64)))
    opt = torch.optim.AdamW([p], lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    w, m, v = w0, np.zeros_like(w0), np.zeros_like(w0)
    for t, gr in enumerate(grads, start=1):
        w, m, v = oracle.adamw(w, gr, m, v, t)
        p.grad = torch.from_numpy(np.clip(gr.astype(np.float64) / 65536, -1, 1))
        opt.step()
    assert_close(w, p.detach().numpy(), rtol=1e-6, atol=1e-7, what="adamw 5 steps")


def test_adamw_first_step_closed_form():
    # step 1: m_hat = g', v_hat = g'^2, so w' = w(1 - lr wd) - lr g' / (|g'| + eps)
    w = np.array([1.0, -2.0, 0.5, 3.0], np.float32)
    gr = np.array([0.25, -5.0, 0.0, 1e-3], np.float32) * 65536
    w1, m1, v1 = oracle.adamw(w, gr, np.zeros(4, np.float32), np.zeros(4, np.float32), 1)
    gc = np.clip(gr.astype(np.float64) / 65536, -1, 1)
    want = w * (1 - 1e-3 * 0.01) - 1e-3 * gc / (np.abs(gc) + 1e-8)
    assert_close(w1, want, rtol=1e-6, atol=1e-9, what="adamw step 1")
    # (1 - beta) is formed in f32: 1 - 0.999f = 0.00099998713..., not 1e-3
    c1 = 1.0 - np.float64(np.float32(0.9))
    c2 = np.float64(np.float32(1.0) - np.float32(0.999))
    assert_close(m1, c1 * gc, rtol=1e-6, atol=0, what="m")
    assert_close(v1, c2 * gc * gc, rtol=1e-6, atol=0, what="v")


def test_adamw_nan_gradient_propagates():
    # Rust's f32::clamp keeps NaN (a min/max clamp would turn it into -1)
    w, m, v = oracle.adamw(np.ones(2, np.float32), np.array([np.nan, 1.0], np.float32),
                           np.zeros(2, np.float32), np.zeros(2, np.float32), 1)
    assert np.isnan(w[0]) and np.isnan(m[0]) and np.isfinite(w[1])


# ---------------------------------------------------------------------------
# RoPE and attention prefill
# ---------------------------------------------------------------------------

def rope64(x, head_dim, pos_offset=0):
    """RoPE in float64 with theta rounded as the reference forms it (f32
    position / f32 powf), so only the rotation itself is float64."""
    x = np.asarray(x, np.float64)
    out = x.copy()
    S = x.shape[-2]
    for i in range(0, head_dim, 2):
        f = np.float32(10000.0) ** (np.float32(i) / np.float32(head_dim))
        pos = (np.arange(S) + pos_offset).astype(np.float32)
        th = (pos / np.float32(f)).astype(np.float64)[:, None]
        for h0 in range(0, x.shape[-1], head_dim):
            x1, x2 = x[..., h0 + i], x[..., h0 + i + 1]
            c, s = np.cos(th[:, 0]), np.sin(th[:, 0])
            out[..., h0 + i] = x1 * c - x2 * s
            out[..., h0 + i + 1] = x1 * s + x2 * c
    return out


def test_rope_against_float64_and_invariants():
    g = rng(80)
    x = g.standard_normal((2, 50, 4 * 16)).astype(np.float32)
    got = oracle.rope(x, 16, pos_offset=7)
    assert_close(got, rope64(x, 16, 7), rtol=1e-5, atol=2e-6, what="rope")
    assert np.array_equal(oracle.rope(x[:, :1], 16, 0), x[:, :1])  # position 0: identity
    # a rotation keeps every pair's norm
    n0 = x[..., 0::2].astype(np.float64) ** 2 + x[..., 1::2].astype(np.float64) ** 2
    n1 = got[..., 0::2].astype(np.float64) ** 2 + got[..., 1::2].astype(np.float64) ** 2
    assert_close(n1, n0, rtol=1e-5, atol=1e-6, what="pair norms")


@pytest.mark.parametrize("causal,use_rope", [(True, True), (True, False), (False, True),
                                             (False, False)])
def test_attention_against_torch_sdpa(causal, use_rope):
    torch = _torch()
    g = rng(81 + 2 * causal + use_rope)
    B, S, H, D = 2, 37, 3, 32
    q, k, v = (g.standard_normal((B, S, H * D)).astype(np.float32) for _ in range(3))
    flags = (oracle.ATTN_CAUSAL if causal else 0) | (oracle.ATTN_ROPE if use_rope else 0)
    got = oracle.attention(q, k, v, H, flags=flags)
    qq, kk = (rope64(x, D) if use_rope else x.astype(np.float64) for x in (q, k))
    to = lambda x: torch.from_numpy(np.ascontiguousarray(
        x.reshape(B, S, H, D).transpose(0, 2, 1, 3)))
    want = torch.nn.functional.scaled_dot_product_attention(
        to(qq), to(kk), to(v.astype(np.float64)), is_causal=causal,
        scale=float(np.float32(1) / np.sqrt(np.float32(D)))).numpy()
    want = want.transpose(0, 2, 1, 3).reshape(B, S, H * D)
    assert_close(got, want, rtol=1e-4, atol=2e-5, what=f"attention causal={causal} rope={use_rope}")


def test_attention_closed_forms():
    g = rng(82)
    S, D = 20, 16
    q, k, v = (g.standard_normal((S, D)).astype(np.float32) for _ in range(3))
    causal = oracle.attention(q, k, v, 1, flags=oracle.ATTN_CAUSAL | oracle.ATTN_ROPE)
    assert np.array_equal(causal[0], v[0])  # the first query sees only key 0
    vc = np.tile(g.standard_normal((1, D)).astype(np.float32), (S, 1))
    assert_close(oracle.attention(q, k, vc, 1), vc, rtol=1e-6, atol=1e-6, what="constant V")
    # q = 0 without rope: uniform weights, the mean of the visible values
    z = oracle.attention(np.zeros_like(q), k, v, 1, flags=oracle.ATTN_CAUSAL)
    want = np.cumsum(v.astype(np.float64), axis=0) / np.arange(1, S + 1)[:, None]
    assert_close(z, want, rtol=1e-5, atol=1e-6, what="q = 0 mean")
    # positions: causal masking compares t + k_pos with s + q_pos
    shifted = oracle.attention(q, k, v, 1, q_pos=5, k_pos=5, flags=oracle.ATTN_CAUSAL)
    assert np.array_equal(shifted, oracle.attention(q, k, v, 1, flags=oracle.ATTN_CAUSAL))
    none = oracle.attention(q, k, v, 1, q_pos=0, k_pos=100, flags=oracle.ATTN_CAUSAL)
    assert np.all(none == 0)  # every key lies in the future
