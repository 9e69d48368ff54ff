"""GPU parity: seeded random attention prefills against the oracle.

Each case draws 1-3 batches, 1-4 heads, head_dim 64 or 128 (the fixed-shape
kernels) or, for the general kernel, one of 16..256 including two that are
not multiples of 4, 1-320 queries and 1-320 keys, every combination of the causal and
RoPE flags, rotation positions q_pos / k_pos in [0, 300] (chunked prefill:
query row i sits at q_pos + i and sees keys at k_pos + j <= q_pos + i), and
the default scale 1/sqrt(D) or an explicit one.  Rows whose keys are all in
the future come out as zeros, as in the fused WGSL step (lazy.rs:4821-4909).
Tolerance as for every attention test: |g - c| <= 1e-5 + 2e-3 |c| against
the f32 CPU restatement.
"""
import numpy as np
import pytest

import oracle
from conftest import assert_close, rng

pytestmark = pytest.mark.gpu


def random_prefill(seed, general=False, head_dim=None):
    g = rng(seed)
    B, H = int(g.integers(1, 4)), int(g.integers(1, 5))
    D = int(g.choice([16, 24, 32, 48, 80, 96, 104, 112, 144, 160, 192, 256, 50, 70])
            if general else g.choice([64, 128]))
    D = head_dim or D
    S, Sk = int(g.integers(1, 321)), int(g.integers(1, 321))
    flags = int(g.integers(0, 4))
    q_pos, k_pos = int(g.integers(0, 301)), int(g.integers(0, 301))
    scale = 0.0 if g.random() < 0.6 else float(np.float32(g.uniform(0.02, 0.3)))
    q = g.standard_normal((B, S, H * D)).astype(np.float32)
    k = g.standard_normal((B, Sk, H * D)).astype(np.float32)
    v = g.standard_normal((B, Sk, H * D)).astype(np.float32)
    return q, k, v, H, q_pos, k_pos, flags, scale


def run_case(hip, seed, general=False, head_dim=None):
    q, k, v, H, q_pos, k_pos, flags, scale = random_prefill(seed, general, head_dim)
    got = hip.flash_attention(hip.tensor(q), hip.tensor(k), hip.tensor(v), H, q_pos, k_pos,
                              flags, scale).numpy()
    want = oracle.attention(q, k, v, H, q_pos, k_pos, flags, scale or None)
    B, S, X = q.shape
    assert_close(got, want, 2e-3, 1e-5,
                 f"seed {seed}: B={B} S={S} Sk={k.shape[1]} H={H} D={X // H} flags={flags} "
                 f"q_pos={q_pos} k_pos={k_pos} scale={scale}")


@pytest.mark.parametrize("seed", range(24))
def test_random_prefill(hip, seed):
    run_case(hip, 700 + seed)


@pytest.mark.parametrize("seed", range(16))
def test_random_prefill_general_head_dims(hip, seed):
    run_case(hip, 800 + seed, general=True)


# Head dims whose 16-query kernel moves 64-key blocks (laid out for 16 or 64
# dims): 16-byte pieces (12, 60) and single floats (14, 62), and the
# fixed-shape 64, each over four seeded shapes and flag sets.
@pytest.mark.parametrize("head_dim", [12, 14, 16, 60, 62, 64])
@pytest.mark.parametrize("seed", range(4))
def test_random_prefill_64_key_blocks(hip, head_dim, seed):
    run_case(hip, 900 + 10 * head_dim + seed, head_dim=head_dim)
