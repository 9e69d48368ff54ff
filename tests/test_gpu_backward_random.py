"""GPU parity: seeded random shapes for the row losses and backward passes.

Each case draws a row count in 1..299 and a width from one of the kernel
families (a wave per row up to 1024 columns, two rows per workgroup up to
4096, a workgroup per row up to 16384 in 4-float vectors, and the loop
kernels past that or at widths that are not a multiple of 4), a count of
targets in 1..rows (rows past it count zero), targets anywhere in the row,
and a random gradient scale; then it runs softmax backward, cross entropy
and its backward, MSE and its backward and the broadcast gradient against
the oracle, at the bounds of the fixed-shape tests in test_gpu_backward.py.
"""
import numpy as np
import pytest

import oracle
from conftest import assert_close, rng
from test_gpu_backward import softmax_bw_check

pytestmark = pytest.mark.gpu


def random_case(seed):
    g = rng(seed)
    rows = int(g.integers(1, 300))
    family = int(g.integers(0, 5))
    cols = int([g.integers(1, 1025), 4 * g.integers(257, 1025), 4 * g.integers(1025, 4097),
                g.integers(16385, 20000), g.integers(1025, 9000)][family])
    used = int(g.integers(1, rows + 1))
    scale = float(np.float32(g.uniform(0.1, 4.0)))
    return g, rows, cols, used, scale


@pytest.mark.parametrize("seed", range(24))
def test_random_losses_and_backward(hip, seed):
    g, rows, cols, used, scale = random_case(1000 + seed)
    what = f"seed {seed}: {rows}x{cols}, {used} targets, scale {scale}"
    logits = g.normal(0, 3, (rows, cols)).astype(np.float32)
    t = g.integers(0, cols, used).astype(np.float32)
    tl, tt = hip.tensor(logits), hip.tensor(t)
    gl = hip.tensor(np.array([scale], np.float32))

    loss = hip.cross_entropy(tl, tt).numpy()[0, 0]
    want = oracle.cross_entropy(logits, t)[0, 0]
    assert abs(loss - want) <= 1e-4 * abs(want) + 1e-7, f"{what}: loss {loss} want {want}"
    grad = hip.cross_entropy_backward(tl, tt, gl).numpy()
    assert_close(grad, oracle.cross_entropy_backward(logits, t, scale), 1e-4,
                 1e-4 * scale / rows * 1e-2, f"{what}: ce backward")
    assert np.all(grad[used:] == 0), f"{what}: rows without a target"

    y = oracle.softmax(logits)
    dy = g.standard_normal((rows, cols)).astype(np.float32)
    got = hip.softmax_backward(hip.tensor(y), hip.tensor(dy)).numpy()
    softmax_bw_check(got, y, dy, f"{what}: softmax backward")

    p = g.standard_normal((rows, cols)).astype(np.float32)
    q = g.standard_normal((rows, cols)).astype(np.float32)
    tp, tq = hip.tensor(p), hip.tensor(q)
    mse = hip.mse(tp, tq).numpy()[0, 0]
    exact = np.mean((p.astype(np.float64) - q) ** 2)
    assert abs(mse - exact) <= 1e-4 * exact, f"{what}: mse {mse} exact {exact}"
    assert_close(hip.mse_backward(tp, tq, gl).numpy(), oracle.mse_backward(p, q, scale), 1e-6,
                 1e-30, f"{what}: mse backward")

    # the broadcast operand gradient of a [rows, cols] output onto [cols]
    gb = hip.broadcast_grad(hip.tensor(dy), cols).numpy()
    want_b = oracle.bias_grad(dy, cols)
    assert np.all(np.abs(gb - want_b) <= 1e-4 * np.abs(want_b) + np.sqrt(rows) * 1e-5), \
        f"{what}: broadcast gradient"
