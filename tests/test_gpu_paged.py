"""GPU parity: PagedAttention decode and its block-table gather.

Tolerance (attention, BASELINE): |g - c| <= 1e-5 + 2e-3 |c| against the f32
CPU restatement; gather indices are compared bit for bit.
"""
import numpy as np
import pytest

import oracle
from clove_amd import workloads
from conftest import assert_close, rng

pytestmark = pytest.mark.gpu

RTOL, ATOL = 2e-3, 1e-5


def make(seed, B, H, D, bs, nb, max_blocks, ctx):
    g = rng(seed)
    kv = g.standard_normal((2, nb, bs, H, D), dtype=np.float32)
    q = g.standard_normal((B, H * D), dtype=np.float32)
    kn = g.standard_normal((B, H * D), dtype=np.float32)
    vn = g.standard_normal((B, H * D), dtype=np.float32)
    bt = g.permutation(nb)[: B * max_blocks].reshape(B, max_blocks).astype(np.int32)
    return q, kn, vn, kv, bt, np.asarray(ctx, np.int32)


def run(hip, q, kn, vn, kv, bt, cl, scale=None):
    t = hip.tensor
    out = hip.paged_attention(t(q), t(kn) if kn is not None else None,
                              t(vn) if vn is not None else None, t(kv), t(bt), t(cl), scale)
    return out.numpy()


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("bs", [8, 16, 32])
def test_head_dims_and_block_sizes(hip, D, bs):
    H, B, max_blocks = 2, 4, 1200 // bs + 1
    ctx = [1, bs, 511 + bs, 1200]
    q, kn, vn, kv, bt, cl = make(D + bs, B, H, D, bs, B * max_blocks + 3, max_blocks, ctx)
    want = oracle.paged_attention(q, None, None, kv, bt, cl).reshape(B, H * D)
    assert_close(run(hip, q, None, None, kv, bt, cl), want, RTOL, ATOL, f"D={D} bs={bs}")


# Head dims and block sizes without a fixed-shape kernel: the general kernel
# (head_dim = dim / num_heads is unrestricted in nn.rs:519 and
# nn/attention.rs:47; the lazy plan takes it from q, lazy.rs:2363-2371).
@pytest.mark.parametrize("D", [32, 80, 96, 112, 160])
@pytest.mark.parametrize("bs", [16, 64])
def test_general_head_dims(hip, D, bs):
    H, B = 3, 4
    ctx = [1, bs + 1, 1500, 2600]
    mb = 2600 // bs + 1
    q, kn, vn, kv, bt, cl = make(1000 + D + bs, B, H, D, bs, B * mb + 2, mb, ctx)
    want = oracle.paged_attention(q, kn, vn, kv, bt, cl).reshape(B, H * D)
    assert_close(run(hip, q, kn, vn, kv, bt, cl), want, RTOL, ATOL, f"D={D} bs={bs} new token")
    want = oracle.paged_attention(q, None, None, kv, bt, cl).reshape(B, H * D)
    assert_close(run(hip, q, None, None, kv, bt, cl), want, RTOL, ATOL, f"D={D} bs={bs} cached")


# Odd shapes: head dims not a multiple of 4 (4-byte loads), a head dim past
# 512 (one register buffer), block sizes 1, 5 and 128, and more heads than a
# multiple of the four per workgroup.
@pytest.mark.parametrize("D,bs,H", [(1, 16, 2), (7, 5, 5), (50, 1, 3), (100, 24, 2),
                                    (300, 128, 1), (520, 16, 2), (1024, 8, 1), (64, 48, 6)])
def test_general_odd_shapes(hip, D, bs, H):
    B = 3
    ctx = [1, 777, 300]
    mb = 777 // bs + 1
    q, kn, vn, kv, bt, cl = make(2000 + D + bs, B, H, D, bs, B * mb + 1, mb, ctx)
    want = oracle.paged_attention(q, kn, vn, kv, bt, cl).reshape(B, H * D)
    assert_close(run(hip, q, kn, vn, kv, bt, cl), want, RTOL, ATOL, f"D={D} bs={bs} H={H}")


@pytest.mark.parametrize("D,bs", [(128, 16), (64, 8), (256, 32)])
def test_general_kernel_at_fixed_shapes(hip, monkeypatch, D, bs):
    # CLOVE_PAGED_GENERAL=1 sends a fixed shape to the general kernel: both
    # must meet the bound, and partitions of 2048 tokens cover several LDS
    # row chunks (512 tokens each)
    H, B = 4, 3
    ctx = [2049, 4096, 513]
    mb = 4096 // bs
    q, kn, vn, kv, bt, cl = make(3000 + D, B, H, D, bs, B * mb + 1, mb, ctx)
    want = oracle.paged_attention(q, kn, vn, kv, bt, cl).reshape(B, H * D)
    tuned = run(hip, q, kn, vn, kv, bt, cl)
    monkeypatch.setenv("CLOVE_PAGED_GENERAL", "1")
    general = run(hip, q, kn, vn, kv, bt, cl)
    assert_close(tuned, want, RTOL, ATOL, "fixed-shape kernel")
    assert_close(general, want, RTOL, ATOL, "general kernel")


@pytest.mark.parametrize("part", [24, 1000, 2052])
def test_general_partitions(hip, monkeypatch, part):
    # partitions that end inside a block and inside an LDS row chunk
    monkeypatch.setenv("CLOVE_PAGED_PART", str(part))
    H, D, bs, B = 2, 96, 12, 3
    ctx = [2053, 1000, 25]
    mb = 2053 // bs + 1
    q, kn, vn, kv, bt, cl = make(4000 + part, B, H, D, bs, B * mb + 3, mb, ctx)
    want = oracle.paged_attention(q, kn, vn, kv, bt, cl).reshape(B, H * D)
    assert_close(run(hip, q, kn, vn, kv, bt, cl), want, RTOL, ATOL, f"part={part}")


# Head pairs: D = 16 or 48 with an even head count runs the general kernel on
# rows of two heads; H = 10 leaves the last workgroup with one of its four
# pairs; small partitions exercise the per-head partials and the merge.  The
# single-head form (CLOVE_PAGED_PAIRS=0) meets the same bound on the same
# inputs.
@pytest.mark.parametrize("D,bs,H,part", [(16, 16, 2, None), (48, 7, 6, None), (48, 16, 10, None),
                                         (16, 64, 4, None), (16, 5, 2, 300), (48, 16, 4, 100)])
def test_general_head_pairs(hip, monkeypatch, D, bs, H, part):
    if part is not None:
        monkeypatch.setenv("CLOVE_PAGED_PART", str(part))
    B = 4
    ctx = [1, bs + 1, 1500, 2600]
    mb = 2600 // bs + 1
    q, kn, vn, kv, bt, cl = make(5000 + D + bs + H, B, H, D, bs, B * mb + 2, mb, ctx)
    want = oracle.paged_attention(q, kn, vn, kv, bt, cl).reshape(B, H * D)
    pairs = run(hip, q, kn, vn, kv, bt, cl)
    assert_close(pairs, want, RTOL, ATOL, f"D={D} bs={bs} H={H} new token")
    monkeypatch.setenv("CLOVE_PAGED_PAIRS", "0")
    single = run(hip, q, kn, vn, kv, bt, cl)
    assert_close(single, want, RTOL, ATOL, f"D={D} bs={bs} H={H} single heads")
    monkeypatch.delenv("CLOVE_PAGED_PAIRS")
    want = oracle.paged_attention(q, None, None, kv, bt, cl).reshape(B, H * D)
    assert_close(run(hip, q, None, None, kv, bt, cl), want, RTOL, ATOL, f"D={D} H={H} cached")


def test_general_bad_table_entry_is_reported_not_read(hip):
    q, kn, vn, kv, bt, cl = make(8, 2, 2, 96, 16, 20, 4, [40, 40])
    bt[1, 1] = 1 << 30
    out = hip.paged_attention(hip.tensor(q), None, None, hip.tensor(kv), hip.tensor(bt),
                              hip.tensor(cl))
    with pytest.raises(hip.CloveError) as e:
        hip.synchronize()
    assert e.value.code == hip.ERR_RANGE
    want = oracle.paged_attention(q[:1], None, None, kv, bt[:1], cl[:1]).reshape(1, 192)
    assert_close(out.numpy()[:1], want, RTOL, ATOL, "unaffected sequence")
    hip.synchronize()


@pytest.mark.parametrize("D,bs,ctx", [(128, 16, [1, 2, 15, 16]), (128, 16, [17, 511, 512, 513]),
                                      (128, 16, [1024, 1535, 2049, 0]),
                                      (256, 32, [1, 16, 17, 32]), (256, 32, [33, 511, 512, 2049])])
def test_context_edges_with_new_token(hip, D, bs, ctx):
    H = 4
    mb = 2560 // bs
    q, kn, vn, kv, bt, cl = make(sum(ctx) + D, 4, H, D, bs, 4 * mb, mb, ctx)
    want = oracle.paged_attention(q, kn, vn, kv, bt, cl).reshape(4, H * D)
    assert_close(run(hip, q, kn, vn, kv, bt, cl), want, RTOL, ATOL, f"ctx={ctx}")
    want = oracle.paged_attention(q, None, None, kv, bt, cl).reshape(4, H * D)
    assert_close(run(hip, q, None, None, kv, bt, cl), want, RTOL, ATOL, f"ctx={ctx} cached")


@pytest.mark.parametrize("part", [2048, 2056, 4096])
def test_long_partitions(hip, monkeypatch, part):
    # Block size 8: a 2048-token partition holds 256 whole blocks, the most
    # the kernel's register-held table covers (the pipelined path); 2056 and
    # 4096 tokens exceed it and take the block-by-block path.  Contexts end
    # on, just before and just after partition boundaries.
    monkeypatch.setenv("CLOVE_PAGED_PART", str(part))
    H, D, bs, B = 2, 64, 8, 4
    ctx = [4103, 2048, 2057, 4096]
    mb = 4104 // bs + 1
    q, kn, vn, kv, bt, cl = make(part, B, H, D, bs, B * mb + 3, mb, ctx)
    want = oracle.paged_attention(q, kn, vn, kv, bt, cl).reshape(B, H * D)
    assert_close(run(hip, q, kn, vn, kv, bt, cl), want, RTOL, ATOL, f"part={part}")


def test_empty_context_writes_zeros(hip):
    q, kn, vn, kv, bt, cl = make(5, 3, 2, 64, 16, 40, 8, [0, 3, 0])
    out = run(hip, q, None, None, kv, bt, cl)
    assert np.all(out[0] == 0) and np.all(out[2] == 0)


def test_explicit_scale(hip):
    q, kn, vn, kv, bt, cl = make(6, 2, 2, 64, 16, 40, 8, [100, 7])
    want = oracle.paged_attention(q, None, None, kv, bt, cl, scale=0.3).reshape(2, 128)
    assert_close(run(hip, q, None, None, kv, bt, cl, 0.3), want, RTOL, ATOL, "scale")


def test_gather_indices_bit_exact(hip):
    g = rng(7)
    bt = g.permutation(5000)[: 8 * 300].reshape(8, 300).astype(np.int32)
    cl = np.array([0, 1, 15, 16, 17, 4095, 4800, 2000], np.int32)
    got = hip.paged_gather_indices(hip.tensor(bt), hip.tensor(cl), 16, 4810).numpy()
    assert np.array_equal(got, oracle.paged_slots(bt, cl, 16, 4810))


def test_bad_table_entry_is_reported_not_read(hip):
    # An entry outside the pool must not be dereferenced; the kernel skips it
    # and the next synchronising call reports CLOVE_HIP_ERR_RANGE.
    q, kn, vn, kv, bt, cl = make(8, 2, 2, 64, 16, 20, 4, [40, 40])
    bt[1, 1] = 1 << 30
    out = hip.paged_attention(hip.tensor(q), None, None, hip.tensor(kv), hip.tensor(bt),
                              hip.tensor(cl))
    with pytest.raises(hip.CloveError) as e:
        hip.synchronize()
    assert e.value.code == hip.ERR_RANGE
    want = oracle.paged_attention(q[:1], None, None, kv, bt[:1], cl[:1]).reshape(1, 128)
    assert_close(out.numpy()[:1], want, RTOL, ATOL, "unaffected sequence")
    hip.synchronize()  # the flag was cleared by the report


def test_shape_errors(hip):
    q, kn, vn, kv, bt, cl = make(9, 2, 1, 1025, 16, 20, 4, [5, 5])
    with pytest.raises(hip.CloveError):  # head_dim above 1024
        run(hip, q, None, None, kv, bt, cl)
    q, kn, vn, kv, bt, cl = make(9, 2, 2, 64, 16, 20, 4, [5, 5])
    with pytest.raises(hip.CloveError):  # q with the wrong element count
        run(hip, q[:, :64], None, None, kv, bt, cl)


@pytest.fixture(scope="module")
def config5(hip):
    """Config 5: B=32, H=32, D=128, block 16, ctx ~ U[512, 4096], tables from
    a seeded permutation of a 16,384-block pool, Q/K/V normal(0,1), seed 4,
    scale 1/sqrt(128).  The 8 GiB pool is filled on the device."""
    P = workloads.PAGED
    B, H, D, bs, nb = P["num_seqs"], P["num_heads"], P["head_dim"], P["block_size"], P["pool_blocks"]
    ctx, bt = workloads.paged_layout(4)
    kv = hip.empty((2, nb, bs, H, D)).fill_normal(4)
    q = rng(4).standard_normal((B, H * D), dtype=np.float32)
    out = hip.paged_attention(hip.tensor(q), None, None, kv, hip.tensor(bt),
                              hip.tensor(ctx)).numpy()
    yield dict(B=B, H=H, D=D, bs=bs, nb=nb, ctx=ctx, bt=bt, kv=kv, q=q, out=out)
    kv.free()


def test_config5_full(hip, config5):
    """Every sequence of config 5 (all heads) against the oracle, in batches
    of 8 sequences on compact copies of the blocks they use (the gather reads
    the same rows, so this equals the full pool)."""
    c = config5
    B, H, D, bs, nb, kv = c["B"], c["H"], c["D"], c["bs"], c["nb"], c["kv"]
    plane, blk = nb * bs * H * D, bs * H * D

    def read_block(p, b):
        return kv.read(p * plane + b * blk, blk).reshape(bs, H, D)

    assert np.all(np.isfinite(c["out"]))
    for lo in range(0, B, 8):
        seqs = list(range(lo, min(B, lo + 8)))
        pool, sbt, scl = workloads.compact_pool(read_block, c["bt"], c["ctx"], seqs, bs)
        want = oracle.paged_attention(c["q"][seqs], None, None, pool, sbt, scl)
        assert_close(c["out"][seqs], want.reshape(len(seqs), H * D), RTOL, ATOL,
                     f"config5 sequences {seqs[0]}..{seqs[-1]}")


def test_config5_gather_indices_bit_exact(hip, config5):
    """The slots of every token of the config-5 tables, bit for bit against
    the integer closed form (lazy.rs:5262-5270)."""
    c = config5
    tbt, tcl = hip.tensor(c["bt"]), hip.tensor(c["ctx"])
    max_ctx = int(c["ctx"].max())
    got = hip.paged_gather_indices(tbt, tcl, c["bs"], max_ctx).numpy()
    want = oracle.paged_slots(c["bt"], c["ctx"], c["bs"], max_ctx)
    assert np.array_equal(got, want)
    # every slot lies in the pool, and the used slots are distinct
    used = got[got >= 0]
    assert used.max() < c["nb"] * c["bs"] and np.unique(used).size == used.size


def test_config5_f32_tables_equal_int32_tables(hip, config5):
    """Clove builds every tensor from a Vec<f32> (backend.rs:176), so
    nn::PagedAttention passes its block tables and context lengths as f32
    tensors (nn.rs:528-546).  At config 5 they give the int32 result bit for
    bit; the -1 padding past each sequence's blocks is never read, so it is
    no error."""
    c = config5
    f32 = lambda a: hip.tensor(np.asarray(a, np.float32), dtype=np.float32)
    out = hip.paged_attention(hip.tensor(c["q"]), None, None, c["kv"], f32(c["bt"]),
                              f32(c["ctx"])).numpy()
    hip.synchronize()  # no index was reported
    assert np.array_equal(out, c["out"])
    got = hip.paged_gather_indices(f32(c["bt"]), f32(c["ctx"]), c["bs"],
                                   int(c["ctx"].max())).numpy()
    assert np.array_equal(got, oracle.paged_slots(c["bt"], c["ctx"], c["bs"],
                                                  int(c["ctx"].max())))


@pytest.mark.parametrize("D,bs,ctx", [(128, 16, [1, 16, 17, 300]), (256, 32, [1, 32, 33, 320]),
                                      (256, 16, [2, 16, 31, 300]), (64, 32, [1, 31, 64, 301])])
def test_kv_append_then_cached_decode_equals_new_token_decode(hip, D, bs, ctx):
    """The append writes k/v at slot ctx-1; decoding from the cache afterwards
    gives exactly the new-token decode (same rows, same order).  A context
    that ends on a block edge folds its last block through the pipelined path
    when cached and through the checked one with the new token, so the two
    paths must round alike (also where a block is folded in two halves,
    head_dim 256 with 32-token blocks)."""
    q, kn, vn, kv, bt, cl = make(10 + D + bs, 4, 4, D, bs, 4 * (320 // bs + 1) + 8,
                                 320 // bs + 1, ctx)
    t = hip.tensor
    tkv, tbt, tcl = t(kv), t(bt), t(cl)
    fresh = hip.paged_attention(t(q), t(kn), t(vn), tkv, tbt, tcl).numpy()
    hip.paged_kv_append(tkv, t(kn), t(vn), tbt, tcl)
    assert np.array_equal(tkv.numpy(), oracle.paged_kv_append(kv, kn, vn, bt, cl))
    cached = hip.paged_attention(t(q), None, None, tkv, tbt, tcl).numpy()
    assert np.array_equal(cached, fresh)


def test_kv_append_skips_empty_and_reports_bad_entries(hip):
    q, kn, vn, kv, bt, cl = make(11, 3, 2, 64, 16, 20, 4, [0, 5, 20])
    t = hip.tensor
    tkv = t(kv)
    hip.paged_kv_append(tkv, t(kn), t(vn), t(bt), t(cl))
    assert np.array_equal(tkv.numpy(), oracle.paged_kv_append(kv, kn, vn, bt, cl))
    bt[2, 1] = -7
    hip.paged_kv_append(tkv, t(kn), t(vn), t(bt), t(cl))
    with pytest.raises(hip.CloveError) as e:
        hip.synchronize()
    assert e.value.code == hip.ERR_RANGE


def f32t(hip, a):
    return hip.tensor(np.asarray(a, np.float32), dtype=np.float32)


@pytest.mark.parametrize("where,value", [
    ("table", 3.5), ("table", -1.0), ("table", float(1 << 24)), ("table", float("nan")),
    ("ctx", 2.5), ("ctx", -1.0), ("ctx", float("inf")),
])
def test_f32_index_values_must_be_integers(hip, where, value):
    """A used table entry or a context length that is not an integer in
    [0, 2^24) is reported as CLOVE_HIP_ERR_RANGE by the next synchronising
    call; that sequence's bad tokens are skipped and the others are exact."""
    q, kn, vn, kv, bt, cl = make(12, 2, 2, 64, 16, 20, 4, [40, 40])
    btf, clf = bt.astype(np.float32), cl.astype(np.float32)
    if where == "table":
        btf[1, 1] = value
    else:
        clf[1] = value
    out = hip.paged_attention(hip.tensor(q), None, None, hip.tensor(kv), f32t(hip, btf),
                              f32t(hip, clf))
    with pytest.raises(hip.CloveError) as e:
        hip.synchronize()
    assert e.value.code == hip.ERR_RANGE and "f32 block_tables/context_lens" in str(e.value)
    want = oracle.paged_attention(q[:1], None, None, kv, bt[:1], cl[:1]).reshape(1, 128)
    assert_close(out.numpy()[:1], want, RTOL, ATOL, "unaffected sequence")
    hip.synchronize()


def test_f32_unused_table_entries_are_not_checked(hip):
    q, kn, vn, kv, bt, cl = make(13, 2, 2, 64, 16, 20, 4, [17, 40])
    btf = bt.astype(np.float32)
    btf[0, 2:] = [0.5, -3.0]          # sequence 0 uses blocks 0 and 1 only
    got = hip.paged_attention(hip.tensor(q), None, None, hip.tensor(kv), f32t(hip, btf),
                              f32t(hip, cl)).numpy()
    hip.synchronize()
    want = run(hip, q, None, None, kv, bt, cl)
    assert np.array_equal(got, want)


def test_f32_tables_in_kv_append_and_graph(hip):
    """The append and the lazy graph's PagedAttention step take f32 tables
    too, with the int32 results."""
    q, kn, vn, kv, bt, cl = make(14, 4, 4, 128, 16, 200, 32, [1, 16, 17, 300])
    t = hip.tensor
    tkv = t(kv)
    hip.paged_kv_append(tkv, t(kn), t(vn), f32t(hip, bt), f32t(hip, cl))
    assert np.array_equal(tkv.numpy(), oracle.paged_kv_append(kv, kn, vn, bt, cl))
    g = hip.Graph()
    ids = [g.input(s) for s in ("4,512", "4,512", "4,512", "2,200,16,4,128", "4,32", "4")]
    y = g.op("paged_attention", *ids)
    m = g.compile([y])
    got = m.execute([t(q), t(kn), t(vn), t(kv), f32t(hip, bt), f32t(hip, cl)])[0].numpy()
    want = run(hip, q, kn, vn, kv, bt, cl)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("entry", [-5, (1 << 31) - 1, (1 << 28)])
def test_gather_indices_bad_entries_give_minus_one(hip, entry):
    """A negative entry, or one whose slots overflow int32, gives -1 (never a
    wrapped or negative slot) and CLOVE_HIP_ERR_RANGE at the next sync."""
    bt = np.array([[3, entry], [4, 5]], np.int32)
    cl = np.array([20, 20], np.int32)
    out = hip.paged_gather_indices(hip.tensor(bt), hip.tensor(cl), 16, 20)
    with pytest.raises(hip.CloveError) as e:
        hip.synchronize()
    assert e.value.code == hip.ERR_RANGE
    got = out.numpy()
    assert np.array_equal(got[0, :16], 48 + np.arange(16))
    assert np.all(got[0, 16:] == -1)
    assert np.array_equal(got[1], oracle.paged_slots(bt[1:], cl[1:], 16, 20)[0])
