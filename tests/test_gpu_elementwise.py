"""GPU parity: eager elementwise ops and fused chains vs the CPU oracle.

Tolerance (elementwise, BASELINE): |g - c| <= 1e-6 + 1e-5 |c|.  Arithmetic
ops are exact (both sides round each IEEE op identically, the device code is
built with -ffp-contract=off); the transcendental ops differ by a few ulp
between the ROCm device library and glibc, and the atol covers outputs that
cancel to ~0 (gelu's 1 + tanh(u) for u << 0).
"""
import numpy as np
import pytest

import oracle
from conftest import assert_close, rng

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-6


@pytest.mark.parametrize("n", [1, 3, 17, 1000, 65537, 1 << 20])
@pytest.mark.parametrize("name", ["relu", "gelu", "sigmoid", "tanh", "sin", "cos"])
def test_unary(hip, name, n):
    x = rng(n).normal(0, 3, n).astype(np.float32)
    got = getattr(hip, name)(hip.tensor(x)).numpy()
    want = getattr(oracle, name)(x)
    if name == "relu":
        assert np.array_equal(got, want)
    else:
        assert_close(got, want, RTOL, ATOL, name)


@pytest.mark.parametrize("nb", [1, 3, 4, 7, 12, 4096, 4099 * 4, None])
@pytest.mark.parametrize("name", ["add", "sub", "mul"])
def test_binary_broadcast(hip, name, nb):
    g = rng(100 + (nb or 0))
    a = g.standard_normal((37, 451), dtype=np.float32)  # 16687 elements
    if nb is None:
        nb = a.size
    b = g.standard_normal(nb, dtype=np.float32)
    got = getattr(hip, name)(hip.tensor(a), hip.tensor(b)).numpy()
    assert np.array_equal(got, getattr(oracle, name)(a, b)), f"{name} nb={nb}"


def test_mul_scalar_and_shapes(hip):
    x = rng(3).standard_normal((2, 3, 5), dtype=np.float32)
    t = hip.mul_scalar(hip.tensor(x), -1.75)
    assert t.shape == (2, 3, 5)
    assert np.array_equal(t.numpy(), oracle.mul_scalar(x, -1.75))


def test_empty_tensor(hip):
    e = hip.empty((0, 4))
    assert hip.relu(e).shape == (0, 4)


def test_kats_on_device(hip):
    a = hip.tensor2d(np.array([[5.0, 3.0]]))
    b = hip.tensor2d(np.array([[2.0, 4.0]]))
    assert np.array_equal(hip.sub(a, b).numpy(), [[3.0, -1.0]])   # engine_tests.rs:697-703
    assert np.array_equal(hip.mul(a, b).numpy(), [[10.0, 12.0]])  # engine_tests.rs:705-706
    z = hip.tensor2d(np.zeros((1, 1)))
    assert abs(hip.sin(z).numpy()[0, 0]) < 1e-6 and abs(hip.cos(z).numpy()[0, 0] - 1) < 1e-6


# ---------------------------------------------------------------------------
# fused chains (Step::Fused)
# ---------------------------------------------------------------------------

CHAIN = [("mul", -1, -2), ("add", 0, -3), ("gelu", 1), ("mul", 2, -4)]


@pytest.mark.parametrize("n", [5, 4096 * 3 + 2])
def test_chain_small(hip, n):
    g = rng(n)
    ins = [g.standard_normal(n, dtype=np.float32) for _ in range(4)]
    (got,) = hip.fused_chain(CHAIN, [hip.tensor(x) for x in ins])
    (want,) = oracle.chain(CHAIN, ins)
    assert_close(got.numpy(), want, RTOL, ATOL, "chain")


def test_chain_config2_full(hip):
    """Config 2: y = gelu(a*b+c)*d over 4 x 16,777,216 normal(0,1), seed 1,
    and the broadcast variant with c = [4096] over a [4096, 4096] view."""
    g = rng(1)
    a, b, c, d = (g.standard_normal((4096, 4096), dtype=np.float32) for _ in range(4))
    ta, tb, tc, td = (hip.tensor(x) for x in (a, b, c, d))
    (got,) = hip.fused_chain(CHAIN, [ta, tb, tc, td])
    (want,) = oracle.chain(CHAIN, [a, b, c, d])
    assert_close(got.numpy(), want, RTOL, ATOL, "config2")
    cb = c[0].copy()
    (got,) = hip.fused_chain(CHAIN, [ta, tb, hip.tensor(cb), td])
    (want,) = oracle.chain(CHAIN, [a, b, cb, d])
    assert_close(got.numpy(), want, RTOL, ATOL, "config2 broadcast")


def test_chain_stores_intermediates(hip):
    g = rng(7)
    x, y = (g.standard_normal(3001, dtype=np.float32) for _ in range(2))
    ops = [("tanh", -1, 0, True), ("scalar_mul", 0, 0, False, 0.5), ("sub", 1, -2, True),
           ("sigmoid", 2), ("relu_grad", -1, 3)]
    got = hip.fused_chain(ops, [hip.tensor(x), hip.tensor(y)])
    assert len(got) == 3
    t = oracle.tanh(x)
    s = oracle.sub(oracle.mul_scalar(t, 0.5), y)
    sg = oracle.sigmoid(s)
    rg = np.where(x > 0, sg, np.float32(0))
    for g_, w, name in zip(got, [t, s, rg], ["tanh", "sub", "relu_grad"]):
        assert_close(g_.numpy(), w, RTOL, ATOL, name)


def test_chain_dropout_flatten_cast(hip):
    x = rng(8).standard_normal(1024, dtype=np.float32)
    ops = [("dropout", -1, 0, 0, 0.25), ("flatten", 0), ("cast", 1)]
    (got,) = hip.fused_chain(ops, [hip.tensor(x)])
    assert np.array_equal(got.numpy(), oracle.chain(ops, [x])[0])


def test_gelu_grad_against_central_difference(hip):
    g = rng(9)
    x = g.normal(0, 2, 5000).astype(np.float32)
    go = g.standard_normal(5000).astype(np.float32)
    (got,) = hip.fused_chain([("gelu_grad", -1, -2)], [hip.tensor(x), hip.tensor(go)])

    def gelu64(v):
        return 0.5 * v * (1 + np.tanh(np.sqrt(2 / np.pi) * (v + 0.044715 * v ** 3)))

    xd, h = x.astype(np.float64), 1e-5
    want = go * (gelu64(xd + h) - gelu64(xd - h)) / (2 * h)
    assert_close(got.numpy(), want, 1e-5, 2e-6, "gelu_grad")


def test_chain_rejects_bad_operands(hip):
    x = hip.tensor(np.ones(4, np.float32))
    with pytest.raises(hip.CloveError):
        hip.fused_chain([("add", -1, 3)], [x])     # forward reference
    with pytest.raises(hip.CloveError):
        hip.fused_chain([("softmax", -1)], [x])    # not elementwise


@pytest.mark.parametrize("shape", [(1, 1), (3, 5), (64, 64), (65, 129), (4096, 17), (1, 4099),
                                   (1000, 1000), (0, 5), (7, 0)])
def test_transpose(hip, shape):
    """backend.rs:2266-2336: [rows, cols] -> [cols, rows], a pure permutation
    (bit-exact)."""
    x = rng(shape[0] * 3 + shape[1]).standard_normal(shape).astype(np.float32)
    t = hip.transpose(hip.tensor(x))
    assert t.shape == (shape[1], shape[0])
    assert np.array_equal(t.numpy(), x.T)


def test_transpose_needs_2d(hip):
    with pytest.raises(hip.CloveError):
        hip.transpose(hip.tensor(np.ones((2, 3, 4), np.float32)))


@pytest.mark.parametrize("shape", [(2, 3, 4), (5,), (1, 1), (4096, 1025), (0, 3)])
def test_flatten(hip, shape):
    """backend.rs:2337-2370: a copy of the data with shape [1, numel]."""
    x = rng(sum(shape) + 11).standard_normal(shape).astype(np.float32)
    t = hip.flatten(hip.tensor(x))
    assert t.shape == (1, x.size)
    assert np.array_equal(t.numpy(), x.reshape(1, -1))


@pytest.mark.parametrize("sa,sb", [((3, 8), (5, 8)), ((2, 7, 16), (2, 9, 16)), ((4, 33), (1, 4, 33)),
                                   ((0, 4), (3, 4)), ((2, 5, 3), (2, 0, 3)), ((64, 4096), (1, 4096))])
def test_concat_seq(hip, sa, sb):
    """backend.rs:1437-1482: per batch, a's rows then b's (bit-exact); a 2-d
    operand is one batch and the result has a's rank."""
    g = rng(len(sa) * 7 + sa[-1])
    a = g.standard_normal(sa).astype(np.float32)
    b = g.standard_normal(sb).astype(np.float32)
    got = hip.concat_seq(hip.tensor(a), hip.tensor(b))
    a3 = a if a.ndim == 3 else a[None]
    b3 = b if b.ndim == 3 else b[None]
    want = np.concatenate([a3, b3], axis=1)
    if a.ndim == 2:
        want = want[0]
    assert got.shape == want.shape
    assert np.array_equal(got.numpy(), want)


def test_concat_seq_shape_errors(hip):
    t = hip.tensor
    with pytest.raises(hip.CloveError):  # hidden sizes differ
        hip.concat_seq(t(np.ones((2, 4), np.float32)), t(np.ones((2, 5), np.float32)))
    with pytest.raises(hip.CloveError):  # batch sizes differ
        hip.concat_seq(t(np.ones((2, 3, 4), np.float32)), t(np.ones((3, 3, 4), np.float32)))
    with pytest.raises(hip.CloveError):  # rank 1
        hip.concat_seq(t(np.ones(4, np.float32)), t(np.ones(4, np.float32)))
