"""GPU parity: seeded random PagedAttention decodes against the oracle.

Each case draws head_dim (64/128/256, or for the general kernel one of
8..320 including non-multiples of 4), block size (8/16/32, or 1..128), 1-6 sequences
of 1-6 heads, context lengths in [0, 2600] with a bias toward block and
partition edges, the new-token path or the cached one, Clove's default
scale or an explicit one, and block tables whose entries may repeat across
sequences (shared prefixes) with -1 past each context.  The pool is the
used blocks plus spares in a seeded order.  These vary the partition plan
(tokens per partition from batch x heads and the longest context) and the
merge.  Tolerance as for every decode: |g - c| <= 1e-5 + 2e-3 |c| against
the f32 CPU restatement (nn.rs:528-546 via backend.rs:176, 249-256).
"""
import numpy as np
import pytest

import oracle
from conftest import assert_close, rng

pytestmark = pytest.mark.gpu

RTOL, ATOL = 2e-3, 1e-5


def random_decode(seed, general=False):
    """Returns (q, k_new, v_new, kv, block_tables, context_lens, scale);
    k_new/v_new and scale may be None.  `general` draws head dims and block
    sizes that have no fixed-shape kernel."""
    g = rng(seed)
    if general:
        D = int(g.choice([8, 24, 32, 40, 48, 80, 96, 100, 112, 160, 192, 320]))
        bs = int(g.choice([1, 4, 12, 16, 64, 128]))
    else:
        D = int(g.choice([64, 128, 256]))
        bs = int(g.choice([8, 16, 32]))
    B, H = int(g.integers(1, 7)), int(g.integers(1, 7))
    ctx = []
    for _ in range(B):
        kind = g.integers(0, 4)
        if kind == 0:
            ctx.append(int(g.integers(0, 2601)))
        elif kind == 1:  # a block edge
            ctx.append(max(0, bs * int(g.integers(0, 2600 // bs + 1)) + int(g.integers(-1, 2))))
        elif kind == 2:  # a power-of-two partition edge
            ctx.append(max(0, int(g.choice([256, 512, 1024, 2048])) + int(g.integers(-1, 2))))
        else:
            ctx.append(int(g.integers(0, 40)))
    ctx = np.asarray(ctx, np.int32)
    need = -(-ctx // bs)
    max_blocks = max(1, int(need.max()))
    spare = int(g.integers(0, 8))
    nb = int(need.sum()) + spare + 1
    order = g.permutation(nb)
    bt = np.full((B, max_blocks), -1, np.int32)
    pos = 0
    for b in range(B):
        n = int(need[b])
        if b and n and g.random() < 0.3:  # share a prefix with sequence 0
            share = min(n, int(need[0]), int(g.integers(1, n + 1)))
            bt[b, :share] = bt[0, :share]
            bt[b, share:n] = order[pos: pos + n - share]
            pos += n - share
        else:
            bt[b, :n] = order[pos: pos + n]
            pos += n
    kv = g.standard_normal((2, nb, bs, H, D), dtype=np.float32)
    q = g.standard_normal((B, H * D), dtype=np.float32)
    kn = vn = None
    if g.random() < 0.5:
        kn = g.standard_normal((B, H * D), dtype=np.float32)
        vn = g.standard_normal((B, H * D), dtype=np.float32)
    scale = None if g.random() < 0.6 else float(np.float32(g.uniform(0.02, 0.3)))
    return q, kn, vn, kv, bt, ctx, scale


def run_case(hip, seed, general=False):
    q, kn, vn, kv, bt, cl, scale = random_decode(seed, general)
    t = hip.tensor
    got = hip.paged_attention(t(q), t(kn) if kn is not None else None,
                              t(vn) if vn is not None else None, t(kv), t(bt), t(cl),
                              scale).numpy()
    want = oracle.paged_attention(q, kn, vn, kv, bt, cl, scale).reshape(got.shape)
    H, D = kv.shape[3], kv.shape[4]
    assert_close(got, want, RTOL, ATOL,
                 f"seed {seed}: B={len(cl)} H={H} D={D} bs={kv.shape[2]} ctx={cl.tolist()} "
                 f"new={kn is not None} scale={scale}")
    # a sequence with no context gives zeros
    assert not np.any(got.reshape(len(cl), -1)[cl == 0])


@pytest.mark.parametrize("seed", range(30))
def test_random_decode(hip, seed):
    run_case(hip, 500 + seed)


@pytest.mark.parametrize("seed", range(24))
def test_random_decode_general_shapes(hip, seed):
    run_case(hip, 900 + seed, general=True)
