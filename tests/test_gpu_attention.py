"""GPU parity: attention prefill (the fused FlashAttention step) and RoPE
vs the oracle.

Tolerances: RoPE 1e-5 relative + 1e-6 absolute (the device sin/cos differ
from glibc's by an ulp or so; theta itself is formed identically);
attention 2e-3 relative + 1e-5 absolute (the attention bound).
"""
import numpy as np
import pytest

import oracle
from conftest import assert_close, rng

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape,head_dim,pos", [((2, 50, 64), 16, 7), ((10, 128), 128, 0),
                                                ((3, 5, 20), 8, 3), ((1, 4096, 128), 128, 0),
                                                # head_dim % 4 != 0 with 16-byte rows (the
                                                # two-entry table path), and with odd-sized
                                                # rows (the pair-at-a-time kernel)
                                                ((3, 7, 12), 6, 5), ((2, 9, 30), 10, 2),
                                                ((2, 3, 44), 6, 1)])
def test_rope(hip, shape, head_dim, pos):
    x = rng(sum(shape)).standard_normal(shape).astype(np.float32)
    got = hip.rope(hip.tensor(x), head_dim, pos).numpy()
    assert_close(got, oracle.rope(x, head_dim, pos), 1e-5, 1e-6 * max(1, shape[-2] / 64),
                 f"rope {shape}")


def test_rope_cached_table_regrows(hip):
    # The (cos, sin) table is cached per head_dim and regrown when a call needs
    # later positions: every call matches the oracle, and a call repeated after
    # the table grew gives the same bits (entries depend on position only).
    x = rng(92).standard_normal((3, 40, 256)).astype(np.float32)
    first = {}
    for pos in (0, 3000, 70000, 3000, 0):
        got = hip.rope(hip.tensor(x), 64, pos).numpy()
        assert_close(got, oracle.rope(x, 64, pos), 1e-5, 1e-6 * max(1, (pos + 40) / 64),
                     f"rope pos={pos}")
        if pos in first:
            assert np.array_equal(got, first[pos]), f"rope pos={pos} changed after regrowth"
        first[pos] = got


CASES = [
    # B, S, Sk, H, D, flags, q_pos, k_pos
    (1, 37, 37, 1, 64, 3, 0, 0),
    (2, 130, 130, 3, 128, 3, 0, 0),
    (1, 256, 256, 4, 64, 1, 0, 0),
    (2, 100, 100, 2, 128, 0, 0, 0),
    (1, 65, 200, 2, 64, 1, 135, 0),   # chunked prefill: 65 new queries after 135 cached keys
    (1, 65, 200, 2, 128, 3, 135, 0),
    (1, 1, 1, 1, 128, 3, 0, 0),
    (1, 33, 31, 2, 64, 2, 0, 0),
    (3, 200, 77, 1, 128, 0, 0, 0),
    # long runs of whole key blocks
    (1, 300, 700, 2, 64, 0, 0, 0),
    (2, 129, 513, 3, 128, 2, 0, 0),
    (1, 512, 512, 2, 128, 1, 0, 0),
    # head dims without a fixed-shape kernel (the general one, tiles padded
    # to the next multiple of 16 or 32): D % 4 == 0 with 16-byte pieces ...
    (1, 130, 130, 2, 80, 3, 0, 0),
    (2, 100, 257, 3, 96, 3, 157, 0),
    (1, 200, 200, 2, 32, 1, 0, 0),
    (1, 77, 140, 2, 112, 2, 0, 30),
    (1, 129, 129, 2, 160, 3, 0, 0),
    (1, 64, 64, 1, 256, 0, 0, 0),
    (2, 50, 60, 3, 16, 3, 5, 0),
    (1, 90, 90, 2, 200, 3, 0, 0),
    # ... and single floats (D % 4 != 0; RoPE needs D even)
    (1, 70, 70, 2, 50, 3, 0, 0),
    (1, 45, 100, 3, 7, 1, 55, 0),
    (2, 33, 33, 1, 130, 2, 0, 0),
    (1, 20, 20, 2, 1, 0, 0, 0),
]


@pytest.mark.parametrize("B,S,Sk,H,D,flags,q_pos,k_pos", CASES)
def test_flash_attention(hip, B, S, Sk, H, D, flags, q_pos, k_pos):
    g = rng(B * 1000 + S * 7 + Sk + H + D + flags)
    q = g.standard_normal((B, S, H * D)).astype(np.float32)
    k = g.standard_normal((B, Sk, H * D)).astype(np.float32)
    v = g.standard_normal((B, Sk, H * D)).astype(np.float32)
    got = hip.flash_attention(hip.tensor(q), hip.tensor(k), hip.tensor(v), H, q_pos, k_pos,
                              flags).numpy()
    want = oracle.attention(q, k, v, H, q_pos, k_pos, flags)
    assert_close(got, want, 2e-3, 1e-5, f"attention {B}x{S}x{Sk}x{H}x{D} flags={flags}")


def test_flash_attention_2d_and_scale_and_errors(hip):
    g = rng(90)
    q, k, v = (g.standard_normal((70, 128)).astype(np.float32) for _ in range(3))
    tq, tk, tv = hip.tensor(q), hip.tensor(k), hip.tensor(v)
    got = hip.flash_attention(tq, tk, tv, 2, flags=3, scale=0.3).numpy()
    assert_close(got, oracle.attention(q, k, v, 2, flags=3, scale=0.3), 2e-3, 1e-5, "2-d")
    # all keys in the future: zeros
    z = hip.flash_attention(tq, tk, tv, 1, q_pos=0, k_pos=100, flags=1).numpy()
    assert np.all(z == 0)
    x = hip.tensor(np.zeros((5, 300), np.float32))
    with pytest.raises(hip.CloveError):  # head_dim above 256
        hip.flash_attention(x, x, x, 1)
    x = hip.tensor(np.zeros((5, 126), np.float32))
    with pytest.raises(hip.CloveError):  # RoPE on an odd head_dim
        hip.flash_attention(x, x, x, 2, flags=2)
    with pytest.raises(hip.CloveError):
        hip.flash_attention(tq, hip.tensor(k[:, :64]), tv, 1)


def test_flash_attention_prefill_4096_sampled(hip):
    """B=1, S=4096, H=32, D=128, causal + RoPE: sampled query rows of every
    head against the oracle (which computes only those rows)."""
    g = rng(91)
    B, S, H, D = 1, 4096, 32, 128
    q, k, v = (g.standard_normal((B, S, H * D)).astype(np.float32) for _ in range(3))
    got = hip.flash_attention(hip.tensor(q), hip.tensor(k), hip.tensor(v), H).numpy()
    for lo, hi in ((0, 2), (127, 130), (2047, 2049), (4094, 4096)):
        want = oracle.attention(q, k, v, H, rows=(lo, hi))
        assert_close(got[:, lo:hi], want[:, lo:hi], 2e-3, 1e-5, f"rows {lo}..{hi}")


@pytest.mark.parametrize("B,S,Sk,H,D,flags,q_pos,k_pos", [(1, 130, 130, 2, 128, 3, 0, 0),
                                                          (2, 65, 200, 3, 64, 2, 135, 0),
                                                          (1, 300, 300, 1, 128, 3, 7, 7),
                                                          (1, 64, 300, 2, 128, 3, 236, 3),
                                                          (2, 100, 333, 3, 64, 3, 400, 167),
                                                          (1, 140, 140, 2, 80, 3, 0, 0),
                                                          (2, 65, 99, 3, 96, 3, 40, 6),
                                                          (1, 70, 70, 2, 50, 3, 9, 9)])
def test_attention_rope_equals_rope_then_attention(hip, B, S, Sk, H, D, flags, q_pos, k_pos):
    """The RoPE flag rotates k in a pass and q inside the kernel; both use the
    RoPE op's arithmetic and table, so the result equals rotating q and k with
    the RoPE op and running attention without the flag, bit for bit."""
    g = rng(95 + S)
    q, k, v = (g.standard_normal((B, n, H * D)).astype(np.float32) for n in (S, Sk, Sk))
    t = hip.tensor
    fused = hip.flash_attention(t(q), t(k), t(v), H, q_pos, k_pos, flags).numpy()
    qr, kr = hip.rope(t(q), D, q_pos), hip.rope(t(k), D, k_pos)
    split = hip.flash_attention(qr, kr, t(v), H, q_pos, k_pos, flags & ~2).numpy()
    assert np.array_equal(fused, split)


def test_exit_without_shutdown_is_clean(hip):
    """A process that uses the RoPE table cache and exits without
    clove_hip_shutdown: the cache's tensors are released by static
    destructors at exit, after (or before) the allocator's own statics;
    the allocator state is never destroyed, so the exit is clean in any
    order of destruction."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = (
        "import sys; sys.path.insert(0, %r)\n"
        "import numpy as np, clove_amd as ca\n"
        "ca.init(0)\n"
        "x = ca.tensor(np.ones((2, 64, 256), np.float32))\n"
        "y = ca.flash_attention(x, x, x, 2)\n"
        "z = ca.rope(x, 128, 5)\n"
        "ca.synchronize()\n"
        "print('ok', flush=True)\n" % root)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip() == "ok", (r.returncode, r.stdout, r.stderr[-2000:])
