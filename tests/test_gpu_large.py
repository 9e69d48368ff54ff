"""GPU parity past the 32-bit ranges: element counts above 2^32 (the fused
chain's 64-bit index and 64-bit `%` broadcast path, the broadcast gradient's
64-bit strip offsets) and row offsets past 2^31 elements (softmax and layer
norm).  Inputs are built on the device (seeded fills, then a chain), and the
checks read back samples and closed forms, so the host never holds the
16 GiB tensors.

  * chain: x[i] = 0 + b1[i % 4096] + b2[i % 4097] over (2^20 + 1) * 4096
    elements; every value is a small integer, so samples around 2^31, 2^32
    and the end are compared bit for bit;
  * broadcast gradient of x to [4096]: column j sums b1[j] over all rows plus
    b2[(j - r) mod 4097] over rows r (4096 = -1 mod 4097), an exact integer
    below 2^24, so any summation order gives the closed form's bits;
  * softmax / layer norm over [2^19 + 3, 4096]: the rows before and after
    element 2^31 and the last row against the oracle, at the bounds of the
    config-3 parity tests.
"""
import numpy as np
import pytest

import oracle
from conftest import assert_close, rng

pytestmark = pytest.mark.gpu

COLS = 4096
WIDE_ROWS = (1 << 20) + 1  # 4,294,971,392 elements: past 2^32
ROW_ROWS = (1 << 19) + 3   # 2,147,495,936 elements: past 2^31


@pytest.fixture
def fresh(hip):
    yield hip
    hip.synchronize()
    hip.empty_cache()


def test_chain_and_broadcast_grad_past_2_32_elements(fresh):
    hip = fresh
    n = WIDE_ROWS * COLS
    assert n > 1 << 32
    g = rng(61)
    b1 = g.integers(0, 2, COLS).astype(np.float32)
    b2 = g.integers(0, 2, COLS + 1).astype(np.float32)
    zeros = hip.empty((WIDE_ROWS, COLS)).fill_uniform(0, 0.0, 0.0)
    (x,) = hip.fused_chain([("add", -1, -2), ("add", 0, -3)],
                           [zeros, hip.tensor(b1), hip.tensor(b2)])
    del zeros
    assert x.numel == n
    for lo in (0, (1 << 31) - 4096, (1 << 32) - 4096, n - 8192):
        idx = np.arange(lo, lo + 8192, dtype=np.int64)
        want = b1[idx % COLS] + b2[idx % (COLS + 1)]
        assert np.array_equal(x.read(lo, 8192), want), f"chain values at {lo}"

    gb = hip.broadcast_grad(x, COLS).numpy().ravel()
    full, rem = divmod(WIDE_ROWS, COLS + 1)
    j = np.arange(COLS)
    tail = np.array([b2[(jj - np.arange(rem)) % (COLS + 1)].sum() for jj in j])
    want = (WIDE_ROWS * b1.astype(np.float64) + full * b2.sum() + tail).astype(np.float32)
    assert np.all(want < (1 << 24))
    assert np.array_equal(gb, want)


@pytest.mark.parametrize("op", ["softmax", "layer_norm"])
def test_rows_past_2_31_elements(fresh, op):
    hip = fresh
    x = hip.empty((ROW_ROWS, COLS)).fill_normal(62, 0.0, 2.0)
    g = rng(63)
    gamma = g.uniform(0.5, 1.5, COLS).astype(np.float32)
    beta = g.uniform(-0.1, 0.1, COLS).astype(np.float32)
    if op == "softmax":
        y = hip.softmax(x)
    else:
        y = hip.layer_norm(x, hip.tensor(gamma), hip.tensor(beta))
    for r in (0, (1 << 19) - 1, 1 << 19, (1 << 19) + 1, ROW_ROWS - 1):
        xr = x.read(r * COLS, COLS).reshape(1, COLS)
        if op == "softmax":
            want = oracle.softmax(xr)
            rtol, atol = 1e-4, 1e-9
        else:
            want = oracle.layer_norm(xr, gamma, beta)
            rtol, atol = 1e-4, 1e-5
        assert_close(y.read(r * COLS, COLS).reshape(1, COLS), want, rtol, atol, f"{op} row {r}")
