"""GPU: the allocation-free paged decode (clove_hip_paged_attention_noalloc)
against the allocating entry (clove_hip_paged_attention_scaled) it shares
kernels with.  Called through the C ABI with raw device pointers; the
results must match bit for bit, on two calls in a row (the second smaller,
so it runs over the scratch array the first one left behind), and against
the oracle within the attention bound."""
import ctypes as C

import numpy as np
import pytest

import oracle
from conftest import assert_close, rng

pytestmark = pytest.mark.gpu


def make(seed, B, H, D, bs, nb, max_blocks, ctx):
    g = rng(seed)
    kv = g.standard_normal((2, nb, bs, H, D), dtype=np.float32)
    q = g.standard_normal((B, H * D), dtype=np.float32)
    kn = g.standard_normal((B, H * D), dtype=np.float32)
    vn = g.standard_normal((B, H * D), dtype=np.float32)
    bt = g.permutation(nb)[: B * max_blocks].reshape(B, max_blocks).astype(np.int32)
    return q, kn, vn, kv, bt, np.asarray(ctx, np.int32)


def noalloc(hip, q, kn, vn, kv, bt, cl, scale):
    """Runs the entry on device copies; returns (status, out or None)."""
    t = hip.tensor
    B, max_blocks = bt.shape
    _, nb, bs, H, D = kv.shape
    tq, tkv, tbt, tcl = t(q), t(kv), t(bt), t(cl)
    tk = t(kn) if kn is not None else None
    tv = t(vn) if vn is not None else None
    out = hip.empty(q.shape)
    ptr = lambda x: C.c_void_p(x.device_ptr) if x is not None else None
    rc = hip.lib().clove_hip_paged_attention_noalloc(
        ptr(tq), ptr(tk), ptr(tv), ptr(tkv), nb, bs, H, D, ptr(tbt), max_blocks, ptr(tcl), B,
        scale, ptr(out))
    return rc, (out.numpy() if rc == 0 else None)


def allocating(hip, q, kn, vn, kv, bt, cl, scale):
    t = hip.tensor
    return hip.paged_attention(t(q), t(kn) if kn is not None else None,
                               t(vn) if vn is not None else None, t(kv), t(bt), t(cl),
                               scale).numpy()


CASES = [
    # seed, B, H, D, bs, nb, max_blocks, ctx, new token
    (1, 8, 8, 128, 16, 8 * 257, 256, [4096, 1, 2049, 700, 4000, 16, 3000, 2048], False),
    (2, 3, 4, 64, 8, 3 * 130, 129, [1000, 5, 1030], True),
    # a head dim and block size without a fixed-shape kernel (the general one)
    (3, 3, 3, 96, 64, 3 * 40 + 2, 40, [2500, 64, 1999], True),
]


def test_noalloc_matches_allocating_entry_twice(hip):
    for seed, B, H, D, bs, nb, mb, ctx, new in CASES:
        q, kn, vn, kv, bt, cl = make(seed, B, H, D, bs, nb, mb, ctx)
        if not new:
            kn = vn = None
        scale = float(1 / np.sqrt(np.float32(D)))
        rc, got = noalloc(hip, q, kn, vn, kv, bt, cl, scale)
        assert rc == 0, hip.last_error()
        want = allocating(hip, q, kn, vn, kv, bt, cl, scale)
        assert np.array_equal(got, want), f"seed {seed}: differs from the allocating entry"
        ref = oracle.paged_attention(q, kn, vn, kv, bt, cl).reshape(B, H * D)
        assert_close(got, ref, 2e-3, 1e-5, f"seed {seed} vs oracle")


def device_free_bytes():
    """hipMemGetInfo's free bytes on the current device."""
    rt = C.CDLL("libamdhip64.so")
    free, total = C.c_size_t(), C.c_size_t()
    assert rt.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


def test_noalloc_allocates_nothing(hip):
    """The entry's defining property: with its inputs resident and every
    kernel it launches already loaded (by the allocating entry), a call
    changes neither the library's reserved bytes nor the device's free
    bytes; again after the allocator's cache is emptied."""
    seed, B, H, D, bs, nb, mb, ctx, _ = CASES[0]
    q, kn, vn, kv, bt, cl = make(seed, B, H, D, bs, nb, mb, ctx)
    scale = float(1 / np.sqrt(np.float32(D)))
    want = allocating(hip, q, None, None, kv, bt, cl, scale)
    t = hip.tensor
    tq, tkv, tbt, tcl = t(q), t(kv), t(bt), t(cl)
    out = hip.empty(q.shape)
    p = lambda x: C.c_void_p(x.device_ptr)
    f = hip.lib().clove_hip_paged_attention_noalloc
    for empty_first in (False, True):
        if empty_first:
            hip.empty_cache()
        hip.synchronize()
        reserved, free = hip.memory_reserved(), device_free_bytes()
        assert f(p(tq), None, None, p(tkv), nb, bs, H, D, p(tbt), mb, p(tcl), B, scale,
                 p(out)) == 0, hip.last_error()
        hip.synchronize()
        assert hip.memory_reserved() == reserved
        assert device_free_bytes() == free
        assert np.array_equal(out.numpy(), want)


def test_noalloc_across_a_stream_switch(hip):
    """Two calls on different streams: the first on the library's stream, the
    second on a caller-owned stream after clove_hip_set_stream, which waits
    for the stream it replaces.  So the second call never overlaps the first
    in the shared scratch array, and both match the allocating entry."""
    rt = C.CDLL("libamdhip64.so")
    stream = C.c_void_p()
    assert rt.hipStreamCreate(C.byref(stream)) == 0
    f = hip.lib().clove_hip_paged_attention_noalloc
    p = lambda x: C.c_void_p(x.device_ptr)
    try:
        outs, wants = [], []
        for i, (seed, B, H, D, bs, nb, mb, ctx, _) in enumerate(CASES[:2]):
            q, kn, vn, kv, bt, cl = make(seed, B, H, D, bs, nb, mb, ctx)
            scale = float(1 / np.sqrt(np.float32(D)))
            wants.append(allocating(hip, q, None, None, kv, bt, cl, scale))
            t = hip.tensor
            tq, tkv, tbt, tcl = t(q), t(kv), t(bt), t(cl)
            out = hip.empty(q.shape)
            if i == 1:
                assert hip.lib().clove_hip_set_stream(stream) == 0
            assert f(p(tq), None, None, p(tkv), nb, bs, H, D, p(tbt), mb, p(tcl), B, scale,
                     p(out)) == 0, hip.last_error()
            outs.append((out, tq, tkv, tbt, tcl))  # keep the inputs alive until read
        for (out, *_), want in zip(outs, wants):
            assert np.array_equal(out.numpy(), want)
    finally:
        hip.lib().clove_hip_set_stream(None)
        rt.hipStreamDestroy(stream)


def test_noalloc_rejects_a_workspace_past_the_scratch(hip):
    # 512 sequences x 32 heads x 2 partitions x (256 + 2) floats = 33.8 MB of
    # partials: more than the 16 MiB array, refused before any launch (the
    # contexts are 0, so nothing would be read or written anyway)
    B, H, D, bs, mb = 512, 32, 256, 16, 256
    t = hip.tensor
    q = hip.empty((B, H * D))
    kv = hip.empty((2, 1, bs, H, D))
    bt = t(np.zeros((B, mb), np.int32))
    cl = t(np.zeros(B, np.int32))
    out = hip.empty((B, H * D))
    p = lambda x: C.c_void_p(x.device_ptr)
    rc = hip.lib().clove_hip_paged_attention_noalloc(p(q), None, None, p(kv), 1, bs, H, D,
                                                     p(bt), mb, p(cl), B, 0.1, p(out))
    assert rc == hip.ERR_SHAPE
    assert "scratch" in hip.last_error()
    hip.synchronize()


def test_noalloc_argument_errors(hip):
    t = hip.tensor
    q = hip.empty((2, 128))
    kv = hip.empty((2, 4, 16, 2, 64))
    bt = t(np.zeros((2, 2), np.int32))
    cl = t(np.array([3, 3], np.int32))
    p = lambda x: C.c_void_p(x.device_ptr)
    f = hip.lib().clove_hip_paged_attention_noalloc
    # head_dim above the largest with a kernel (1024)
    assert f(p(q), None, None, p(kv), 4, 16, 1, 1025, p(bt), 2, p(cl), 2, 0.1, p(q)) == hip.ERR_SHAPE
    # k without v
    assert f(p(q), p(q), None, p(kv), 4, 16, 2, 64, p(bt), 2, p(cl), 2, 0.1, p(q)) == hip.ERR_INVALID
    # a misaligned pointer
    mis = C.c_void_p(q.device_ptr + 4)
    assert f(mis, None, None, p(kv), 4, 16, 2, 64, p(bt), 2, p(cl), 2, 0.1, p(q)) == hip.ERR_INVALID
    # no sequences: nothing to do
    assert f(None, None, None, None, 4, 16, 2, 64, None, 2, None, 0, 0.1, None) == 0
