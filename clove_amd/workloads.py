"""Synthetic workloads of the benchmark configurations.

Clove's RNG is unseeded (backend.rs:965-974), so every input here comes from
a documented generator: numpy's PCG64 for host-built arrays and the
library's splitmix64 stream (clove_hip_tensor_fill_*) for device-built ones.
The same bytes go to the HIP backend and to the CPU oracle.
"""
from __future__ import annotations

import numpy as np


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


# Config 1 ------------------------------------------------------------------

def mlp_inputs(seed: int = 0):
    """x [64,784] U[0,1); W1 [784,128], W2 [128,10] Kaiming-uniform
    U(+-sqrt(6/fan_in)); b1 [1,128], b2 [1,10] with fan_in = 1, the fan-in
    Clove's Linear gives its bias (nn.rs:111: kaiming_random(1, out)).
    Clove's kaiming_random is a normal with std sqrt(2/fan_in)
    (backend.rs:965-974); the configuration asks for the uniform form."""
    g = rng(seed)
    x = g.random((64, 784), dtype=np.float32)

    def ku(fan_in, shape):
        bound = np.sqrt(6.0 / fan_in)
        return g.uniform(-bound, bound, shape).astype(np.float32)

    return x, ku(784, (784, 128)), ku(1, (1, 128)), ku(128, (128, 10)), ku(1, (1, 10))


# Config 5 ------------------------------------------------------------------

PAGED = dict(num_seqs=32, num_heads=32, head_dim=128, block_size=16, pool_blocks=16384,
             ctx_lo=512, ctx_hi=4096)


def paged_layout(seed: int = 4, num_seqs: int = 32, block_size: int = 16,
                 pool_blocks: int = 16384, ctx_lo: int = 512, ctx_hi: int = 4096):
    """Context lengths uniform in [ctx_lo, ctx_hi] and block tables drawn from
    a seeded Fisher-Yates permutation of the pool: the first
    sum(ceil(ctx_b / block_size)) blocks of the permutation are handed out in
    sequence order.  Unused table entries are -1 (never read).
    Returns (context_lens int32 [B], block_tables int32 [B, max_blocks])."""
    g = rng(seed)
    ctx = g.integers(ctx_lo, ctx_hi + 1, num_seqs).astype(np.int32)
    max_blocks = -(-ctx_hi // block_size)
    perm = np.arange(pool_blocks, dtype=np.int64)
    for i in range(pool_blocks - 1, 0, -1):  # Fisher-Yates, explicit for the record
        j = int(g.integers(0, i + 1))
        perm[i], perm[j] = perm[j], perm[i]
    need = -(-ctx // block_size)
    assert need.sum() <= pool_blocks
    bt = np.full((num_seqs, max_blocks), -1, np.int32)
    pos = 0
    for b in range(num_seqs):
        bt[b, : need[b]] = perm[pos: pos + need[b]]
        pos += int(need[b])
    return ctx, bt


def paged_bytes(ctx: np.ndarray, num_heads: int, head_dim: int, block_size: int,
                with_new: bool = False) -> int:
    """Algorithmic HBM bytes of one decode: every context token's K and V
    head rows once, q and out, the block-table entries used and the context
    lengths (with_new: the new token's k/v replace one cached row each)."""
    row = num_heads * head_dim * 4
    B = ctx.size
    tokens = int(ctx.sum())
    blocks = int((-(-ctx // block_size)).sum())
    return tokens * row * 2 + 2 * B * row + 4 * blocks + 4 * B


def compact_pool(read_block, bt: np.ndarray, ctx: np.ndarray, seqs, block_size: int):
    """Builds a small pool holding only the blocks that sequences `seqs` use,
    with a renumbered table.  `read_block(plane, blk)` returns one block
    [block_size, H, D].  Attention over the compact pool equals attention
    over the full pool bit for bit (the gather reads the same rows)."""
    used = []
    for b in seqs:
        used.extend(int(x) for x in bt[b, : -(-int(ctx[b]) // block_size)])
    remap = {blk: i for i, blk in enumerate(dict.fromkeys(used))}
    first = read_block(0, used[0])
    pool = np.empty((2, len(remap)) + first.shape, np.float32)
    for blk, i in remap.items():
        pool[0, i] = read_block(0, blk)
        pool[1, i] = read_block(1, blk)
    sub_bt = np.full((len(seqs), bt.shape[1]), -1, np.int32)
    for r, b in enumerate(seqs):
        n = -(-int(ctx[b]) // block_size)
        sub_bt[r, :n] = [remap[int(x)] for x in bt[b, :n]]
    return pool, sub_bt, ctx[list(seqs)].copy()
