"""GPU parity: row softmax and layer norm vs the CPU oracle.

Tolerance (reductions, BASELINE): |g - c| <= atol + 1e-4 |c|.  The CPU sums
each row sequentially in f32 and the GPU with a wave64 butterfly; both stay
well inside 1e-4 relative.  atol: 1e-9 for softmax (outputs are >= 0 and
tiny values carry their own relative error), 1e-5 for layer norm (outputs
cancel to ~0 after beta, on an O(1) scale).
"""
import numpy as np
import pytest

import oracle
from conftest import assert_close, rng

pytestmark = pytest.mark.gpu

SHAPES = [(1, 1), (3, 10), (7, 33), (5, 4), (9, 256), (33, 4096), (6, 4100), (2, 8192),
          (3, 16384), (2, 3, 64)]


@pytest.mark.parametrize("shape", SHAPES)
def test_softmax(hip, shape):
    x = rng(sum(shape)).normal(0, 2, shape).astype(np.float32)
    got = hip.softmax(hip.tensor(x))
    assert got.shape == shape
    assert_close(got.numpy(), oracle.softmax(x), 1e-4, 1e-9, f"softmax {shape}")


@pytest.mark.parametrize("shape", SHAPES)
def test_layer_norm(hip, shape):
    g = rng(sum(shape) + 1)
    x = g.normal(0, 2, shape).astype(np.float32)
    cols = shape[-1]
    gam = g.uniform(0.5, 1.5, cols).astype(np.float32)
    bet = g.uniform(-0.1, 0.1, cols).astype(np.float32)
    got = hip.layer_norm(hip.tensor(x), hip.tensor(gam), hip.tensor(bet))
    assert_close(got.numpy(), oracle.layer_norm(x, gam, bet), 1e-4, 1e-5, f"layer_norm {shape}")


# Rows wider than 1024 columns (width a multiple of 4) take one workgroup of
# 512 threads per row with P = 1..16 vectors per thread; these widths hit
# every P, the edges between them and the widths either side of the switch.
WIDE = [1024, 1028, 2048, 2052, 4100, 8192, 8196, 12000, 16384, 32768, 32772]


@pytest.mark.parametrize("cols", WIDE)
def test_wide_rows(hip, cols):
    g = rng(cols)
    x = g.normal(0, 2, (3, cols)).astype(np.float32)
    assert_close(hip.softmax(hip.tensor(x)).numpy(), oracle.softmax(x), 1e-4, 1e-9,
                 f"softmax 3x{cols}")
    gam = g.uniform(0.5, 1.5, cols).astype(np.float32)
    bet = g.uniform(-0.1, 0.1, cols).astype(np.float32)
    got = hip.layer_norm(hip.tensor(x), hip.tensor(gam), hip.tensor(bet)).numpy()
    assert_close(got, oracle.layer_norm(x, gam, bet), 1e-4, 1e-5, f"layer_norm 3x{cols}")


def test_config3_full(hip):
    """Config 3: [8192, 4096] normal(0, 2), seed 2; gamma U[0.5, 1.5],
    beta U[-0.1, 0.1]."""
    g = rng(2)
    x = g.normal(0, 2, (8192, 4096)).astype(np.float32)
    gam = g.uniform(0.5, 1.5, 4096).astype(np.float32)
    bet = g.uniform(-0.1, 0.1, 4096).astype(np.float32)
    tx = hip.tensor(x)
    assert_close(hip.softmax(tx).numpy(), oracle.softmax(x), 1e-4, 1e-9, "softmax config3")
    assert_close(hip.layer_norm(tx, hip.tensor(gam), hip.tensor(bet)).numpy(),
                 oracle.layer_norm(x, gam, bet), 1e-4, 1e-5, "layer_norm config3")


def test_closed_forms_on_device(hip):
    c = hip.softmax(hip.tensor(np.full((4, 4096), -2.5, np.float32))).numpy()
    assert np.all(c == np.float32(1 / 4096))
    beta = np.linspace(-1, 1, 512, dtype=np.float32)
    ln = hip.layer_norm(hip.tensor(np.full((3, 512), 4.0, np.float32)),
                        hip.tensor(np.ones(512, np.float32)), hip.tensor(beta)).numpy()
    assert np.array_equal(ln, np.broadcast_to(beta, ln.shape))


def test_layer_norm_short_gamma_rejected(hip):
    x = hip.tensor(np.ones((2, 8), np.float32))
    with pytest.raises(hip.CloveError):
        hip.layer_norm(x, hip.tensor(np.ones(4, np.float32)), hip.tensor(np.ones(8, np.float32)))


def special_rows(cols, seed):
    """Rows a softmax must keep finite by subtracting the row max (entries of
    +-1000 and 88.7, past exp's range), rows with -inf entries (masked
    positions), and rows whose result is NaN in the reference (all -inf, a
    +inf entry, a NaN entry)."""
    g = rng(seed)
    x = g.normal(0, 2, (8, cols)).astype(np.float32)
    x[0, ::3] = 1000.0
    x[1, :] = -1000.0
    x[1, cols // 2] = -999.0
    x[2, ::2] = 88.7
    x[3, 1::2] = -np.inf
    x[4, :] = -np.inf
    x[5, cols - 1] = np.inf
    x[6, cols // 3] = np.nan
    return x


@pytest.mark.parametrize("cols", [64, 1000, 4096])
def test_softmax_special_values(hip, cols):
    x = special_rows(cols, cols)
    got = hip.softmax(hip.tensor(x)).numpy()
    want = oracle.softmax(x)
    assert np.array_equal(np.isnan(got), np.isnan(want)), f"softmax {cols}: NaN positions"
    ok = ~np.isnan(want)
    assert_close(got[ok], want[ok], 1e-4, 1e-9, f"softmax special rows x{cols}")
    assert np.all(got[3, 1::2] == 0.0)  # masked entries are exactly zero


@pytest.mark.parametrize("cols", [64, 1000, 4096])
def test_layer_norm_offset_and_tiny_rows(hip, cols):
    """Rows on a common offset (mean 3, spread 1: the two-pass variance keeps
    the offset out of the spread) and rows on a tiny scale (spread 1e-3, a
    variance of 1e-6 below eps = 1e-5, so eps sets the scale)."""
    g = rng(cols + 7)
    x = np.concatenate([3.0 + g.normal(0, 1, (4, cols)),
                        g.normal(0, 1e-3, (4, cols))]).astype(np.float32)
    gam = g.uniform(0.5, 1.5, cols).astype(np.float32)
    bet = g.uniform(-0.1, 0.1, cols).astype(np.float32)
    got = hip.layer_norm(hip.tensor(x), hip.tensor(gam), hip.tensor(bet)).numpy()
    assert_close(got, oracle.layer_norm(x, gam, bet), 1e-4, 1e-5, f"layer_norm rows x{cols}")


@pytest.mark.parametrize("seed", range(24))
def test_random_rows(hip, seed):
    """Seeded shapes across the kernel families: widths up to 1024 (a wave
    per row), multiples of 4 up to 32768 (a workgroup per row, every vector
    count), and other widths past 1024 (the loop kernels); rows 1-299."""
    g = rng(3000 + seed)
    rows = int(g.integers(1, 300))
    cols = int([g.integers(1, 1025), 4 * g.integers(257, 8193), g.integers(1025, 20000)][
        int(g.integers(0, 3))])
    x = g.normal(0, 2, (rows, cols)).astype(np.float32)
    what = f"seed {seed}: {rows}x{cols}"
    assert_close(hip.softmax(hip.tensor(x)).numpy(), oracle.softmax(x), 1e-4, 1e-9,
                 f"softmax {what}")
    gam = g.uniform(0.5, 1.5, cols).astype(np.float32)
    bet = g.uniform(-0.1, 0.1, cols).astype(np.float32)
    got = hip.layer_norm(hip.tensor(x), hip.tensor(gam), hip.tensor(bet)).numpy()
    assert_close(got, oracle.layer_norm(x, gam, bet), 1e-4, 1e-5, f"layer_norm {what}")
