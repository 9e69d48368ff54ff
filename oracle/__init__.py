"""oracle -- TEST INFRASTRUCTURE: the CPU restatement of Clove's Rayon kernels.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
may import this package, and only as the checker (or the timed CPU
baseline), never as the thing measured or shipped.  The product path
(clove_amd / libclove_hip.so) never loads it.

Each function wraps one C function of ``clove_oracle.c`` and names the
reference lines it restates.  Parity of the restatement itself is pinned by
tests/test_oracle.py (Clove's own known-answer tests, independent float64
library implementations, closed forms and brute force).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libclove_oracle.so")
_lib: Optional[C.CDLL] = None


def build(force: bool = False) -> None:
    """Compiles clove_oracle.c with the rounding-preserving flags."""
    args = ["make", "-C", _HERE]
    if force:
        args.insert(1, "-B")
    subprocess.run(args, check=True, stdout=subprocess.DEVNULL)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        fp, sz = C.POINTER(C.c_float), C.c_size_t
        i32p = C.POINTER(C.c_int32)
        for name in ("oracle_add", "oracle_sub", "oracle_mul"):
            getattr(L, name).argtypes = [fp, sz, fp, sz, fp]
        L.oracle_mul_scalar.argtypes = [fp, sz, C.c_float, fp]
        for name in ("oracle_relu", "oracle_gelu", "oracle_sigmoid", "oracle_tanh",
                     "oracle_sin", "oracle_cos"):
            getattr(L, name).argtypes = [fp, sz, fp]
        L.oracle_softmax.argtypes = [fp, sz, sz, fp]
        L.oracle_layer_norm.argtypes = [fp, sz, sz, fp, fp, fp]
        L.oracle_matmul.argtypes = [fp, fp, sz, sz, sz, fp]
        L.oracle_matmul_rows.argtypes = [fp, fp, sz, sz, sz, sz, sz, fp]
        L.oracle_paged_attention_f32.argtypes = [fp, fp, fp, fp, C.c_int64, i32p, C.c_int, i32p,
                                                 C.c_int, C.c_int, C.c_int, C.c_int, C.c_float,
                                                 C.c_int, C.c_int, fp]
        L.oracle_paged_attention_f64.argtypes = [fp, fp, fp, fp, C.c_int64, i32p, C.c_int, i32p,
                                                 C.c_int, C.c_int, C.c_int, C.c_int, C.c_float,
                                                 C.POINTER(C.c_double)]
        L.oracle_paged_slots.argtypes = [i32p, C.c_int, i32p, C.c_int, C.c_int, C.c_int, i32p]
        L.oracle_relu_backward.argtypes = [fp, fp, sz, fp]
        L.oracle_gelu_backward.argtypes = [fp, fp, sz, fp]
        L.oracle_softmax_backward.argtypes = [fp, fp, sz, sz, fp]
        L.oracle_matmul_backward_rows.argtypes = [fp, fp, fp, sz, sz, sz, sz, sz, sz, sz, fp, fp]
        L.oracle_bias_grad.argtypes = [fp, sz, sz, C.c_int, fp]
        L.oracle_cross_entropy.argtypes = [fp, fp, sz, sz, sz, fp]
        L.oracle_cross_entropy.restype = C.c_int
        L.oracle_cross_entropy_backward.argtypes = [fp, fp, sz, sz, sz, C.c_float, fp]
        L.oracle_cross_entropy_backward.restype = C.c_int
        L.oracle_mse.argtypes = [fp, fp, sz]
        L.oracle_mse.restype = C.c_float
        L.oracle_mse_backward.argtypes = [fp, fp, sz, C.c_float, fp]
        L.oracle_adamw.argtypes = [fp, fp, fp, fp, sz, C.c_float, C.c_float, C.c_float, C.c_float,
                                   C.c_float, C.c_float, C.c_float, C.c_uint32]
        L.oracle_rope.argtypes = [fp, sz, sz, sz, sz, sz, fp]
        L.oracle_attention.argtypes = [fp, fp, fp, sz, sz, sz, sz, sz, C.c_long, C.c_long, C.c_int,
                                       C.c_float, sz, sz, fp]
        L.oracle_threads.restype = C.c_int
        L.oracle_set_threads.argtypes = [C.c_int]
        _lib = L
    return _lib


def _f(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _i(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_int32))


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def threads() -> int:
    return lib().oracle_threads()


def set_threads(n: int) -> None:
    lib().oracle_set_threads(int(n))


def _binary(name, a, b):
    a, b = _f32(a), _f32(b)
    out = np.empty_like(a)
    getattr(lib(), name)(_f(a), a.size, _f(b), b.size, _f(out))
    return out


def add(a, b):
    """backend.rs:1483-1493: a[i] + b[i % len(b)]."""
    return _binary("oracle_add", a, b)


def sub(a, b):
    """backend.rs:1748-1758: a[i] - b[i % len(b)]."""
    return _binary("oracle_sub", a, b)


def mul(a, b):
    """backend.rs:1598-1617 (scalar b) and the WGSL b[i % len(b)] (:1623)."""
    return _binary("oracle_mul", a, b)


def mul_scalar(a, s: float):
    """backend.rs:1686-1697."""
    a = _f32(a)
    out = np.empty_like(a)
    lib().oracle_mul_scalar(_f(a), a.size, float(s), _f(out))
    return out


def _unary(name, a):
    a = _f32(a)
    out = np.empty_like(a)
    getattr(lib(), name)(_f(a), a.size, _f(out))
    return out


def relu(a):
    """backend.rs:1815-1826."""
    return _unary("oracle_relu", a)


def gelu(a):
    """backend.rs:1917-1928 (tanh form, sqrt(2/pi) in f32)."""
    return _unary("oracle_gelu", a)


def sigmoid(a):
    """backend.rs:2951-2960."""
    return _unary("oracle_sigmoid", a)


def tanh(a):
    """backend.rs:3008-3016."""
    return _unary("oracle_tanh", a)


def sin(a):
    """backend.rs:1986-1997."""
    return _unary("oracle_sin", a)


def cos(a):
    """backend.rs:2044-2055."""
    return _unary("oracle_cos", a)


def softmax(a):
    """backend.rs:2102-2125, rows over the last dimension."""
    a = _f32(a)
    cols = a.shape[-1]
    out = np.empty_like(a)
    lib().oracle_softmax(_f(a), a.size // cols if cols else 0, cols, _f(out))
    return out


def layer_norm(a, gamma, beta):
    """backend.rs:2380-2405, rows over the last dimension, eps 1e-5."""
    a, g, b = _f32(a), _f32(gamma), _f32(beta)
    cols = a.shape[-1]
    out = np.empty_like(a)
    lib().oracle_layer_norm(_f(a), a.size // cols if cols else 0, cols, _f(g), _f(b), _f(out))
    return out


def matmul(a, b, rows: Optional[tuple] = None):
    """backend.rs:266-287 (rayon_matmul) with m = prod(a.shape[:-1]).

    ``rows=(r0, r1)`` computes only those output rows (others are zero).
    """
    a, b = _f32(a), _f32(b)
    k = a.shape[-1]
    m = a.size // k if k else 0
    n = b.shape[1]
    out = np.zeros(a.shape[:-1] + (n,), dtype=np.float32)
    r0, r1 = rows if rows is not None else (0, m)
    lib().oracle_matmul_rows(_f(a), _f(b), m, k, n, r0, r1, _f(out))
    return out


def paged_attention(q, k_new, v_new, kv_cache, block_tables, context_lens, scale=None,
                    seqs: Optional[tuple] = None, f64: bool = False):
    """Textbook paged decode on Clove's cache layout (nn.rs:534-535).

    kv_cache is [2, num_blocks, block_size, H, D] (planes K, V).  When
    k_new/v_new are given, token ctx-1 comes from them.  ``f64`` returns the
    float64 evaluation; ``seqs=(s0, s1)`` restricts the f32 evaluation to
    those sequences (other rows stay zero).
    """
    kv = _f32(kv_cache)
    _, nb, bs, H, D = kv.shape
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    cl = np.ascontiguousarray(context_lens, dtype=np.int32)
    B = cl.size
    q = _f32(q).reshape(B, H, D)
    kn = _f32(k_new).reshape(B, H, D) if k_new is not None else None
    vn = _f32(v_new).reshape(B, H, D) if v_new is not None else None
    if scale is None:
        scale = 1.0 / np.sqrt(np.float32(D))
    null = C.POINTER(C.c_float)()
    if f64:
        out = np.zeros((B, H, D), dtype=np.float64)
        lib().oracle_paged_attention_f64(
            _f(q), _f(kn) if kn is not None else null, _f(vn) if vn is not None else null,
            _f(kv), nb, _i(bt), bt.shape[1], _i(cl), B, H, D, bs, float(scale),
            out.ctypes.data_as(C.POINTER(C.c_double)))
        return out
    out = np.zeros((B, H, D), dtype=np.float32)
    s0, s1 = seqs if seqs is not None else (0, B)
    lib().oracle_paged_attention_f32(
        _f(q), _f(kn) if kn is not None else null, _f(vn) if vn is not None else null,
        _f(kv), nb, _i(bt), bt.shape[1], _i(cl), B, H, D, bs, float(scale), s0, s1, _f(out))
    return out


def paged_kv_append(kv_cache, k_new, v_new, block_tables, context_lens):
    """Copy of kv_cache with each sequence's new-token k/v written at the slot
    of token ctx-1 (the cache write that precedes decode; Clove has none).
    Sequences with ctx <= 0 are left alone."""
    kv = np.array(kv_cache, dtype=np.float32, copy=True)
    _, nb, bs, H, D = kv.shape
    bt = np.asarray(block_tables, dtype=np.int64)
    cl = np.asarray(context_lens, dtype=np.int64)
    kn = np.asarray(k_new, dtype=np.float32).reshape(cl.size, H, D)
    vn = np.asarray(v_new, dtype=np.float32).reshape(cl.size, H, D)
    for b in range(cl.size):
        t = int(cl[b]) - 1
        if t < 0:
            continue
        blk = int(bt[b, t // bs])
        kv[0, blk, t % bs] = kn[b]
        kv[1, blk, t % bs] = vn[b]
    return kv


def paged_slots(block_tables, context_lens, block_size: int, max_ctx: int):
    """Physical slot of each logical token (lazy.rs:5262-5270), -1 past ctx."""
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    cl = np.ascontiguousarray(context_lens, dtype=np.int32)
    out = np.empty((cl.size, max_ctx), dtype=np.int32)
    lib().oracle_paged_slots(_i(bt), bt.shape[1], _i(cl), cl.size, block_size, max_ctx, _i(out))
    return out


# ---------------------------------------------------------------------------
# compositions (the eager CPU path runs each op as its own pass)
# ---------------------------------------------------------------------------

_EW = {
    "add": add, "sub": sub, "mul": mul, "relu": relu, "gelu": gelu, "sigmoid": sigmoid,
    "tanh": tanh, "sin": sin, "cos": cos,
}


def chain(ops, inputs):
    """Evaluates a fused-chain description op by op, materialising every
    value in f32 exactly as the eager CPU path would (one pass per op).

    ``ops`` uses the clove_amd.fused_chain tuple format.  Returns the values
    of the stored ops (the last op always), in op order.
    """
    vals = []
    outs = []

    def get(src):
        return vals[src] if src >= 0 else _f32(inputs[-src - 1])

    for i, op in enumerate(ops):
        name, s0, s1, store, param = (tuple(op) + (0, 0, 0, 0.0))[:5]
        name = name.lower()
        if name in ("add", "sub", "mul"):
            a = get(s0)
            v = _EW[name](a, get(s1))
        elif name == "scalar_mul":
            v = mul_scalar(get(s0), param)
        elif name == "dropout":
            v = mul_scalar(get(s0), np.float32(1.0) / (np.float32(1.0) - np.float32(param)))
        elif name in ("flatten", "cast"):
            v = get(s0).copy()
        else:
            v = _EW[name](get(s0))
        vals.append(v)
        if store or i + 1 == len(ops):
            outs.append(v)
    return outs


def mlp_forward(x, w1, b1, w2, b2):
    """Config 1: softmax(relu(x.W1 + b1).W2 + b2) through Linear::forward
    (nn.rs:115-118: matmul then add with b[i % out]), relu and softmax."""
    h = relu(add(matmul(x, w1), b1))
    return softmax(add(matmul(h, w2), b2))


# ---------------------------------------------------------------------------
# backward passes and losses
# ---------------------------------------------------------------------------

def relu_backward(x, g):
    """backend.rs:1858-1870: g where relu's output (equivalently x) > 0."""
    x, g = _f32(x), _f32(g)
    out = np.empty_like(x)
    lib().oracle_relu_backward(_f(x), _f(g), x.size, _f(out))
    return out


def gelu_backward(x, g):
    """backend.rs:1965-1981: g times the tanh-form GELU derivative."""
    x, g = _f32(x), _f32(g)
    out = np.empty_like(x)
    lib().oracle_gelu_backward(_f(x), _f(g), x.size, _f(out))
    return out


def softmax_backward(y, dy):
    """backend.rs:2163-2183: dx = y * (dy - sum(dy * y)) per row."""
    y, dy = _f32(y), _f32(dy)
    cols = y.shape[-1]
    out = np.empty_like(y)
    lib().oracle_softmax_backward(_f(y), _f(dy), y.size // cols, cols, _f(out))
    return out


def matmul_backward(a, b, dc, da_rows: Optional[tuple] = None, db_rows: Optional[tuple] = None):
    """backend.rs:1314-1360: dA = dC . B^T and dB = A^T . dC as sequential
    f32 dots.  da_rows / db_rows restrict the computed rows (others stay 0)."""
    a, b, dc = _f32(a), _f32(b), _f32(dc)
    k = a.shape[-1]
    m = a.size // k
    n = b.shape[1]
    da = np.zeros((m, k), np.float32)
    db = np.zeros((k, n), np.float32)
    r0, r1 = da_rows or (0, m)
    s0, s1 = db_rows or (0, k)
    lib().oracle_matmul_backward_rows(_f(a), _f(b), _f(dc), m, k, n, r0, r1, s0, s1, _f(da), _f(db))
    return da.reshape(a.shape), db


def bias_grad(g, nb: int, negate: bool = False):
    """backend.rs:1527-1538 (add) / 1800-1810 (sub): the b operand's gradient,
    gb[i % nb] (+/-)= g[i] folded in index order."""
    g = _f32(g)
    out = np.empty(nb, np.float32)
    lib().oracle_bias_grad(_f(g), g.size, nb, int(negate), _f(out))
    return out


def cross_entropy(logits, targets):
    """backend.rs:2661-2680: mean over rows of logsumexp(row) - row[target]."""
    l, t = _f32(logits), _f32(targets)
    out = np.zeros(1, np.float32)
    cols = l.shape[-1]
    if lib().oracle_cross_entropy(_f(l), _f(t), t.size, l.size // cols, cols, _f(out)) != 0:
        raise IndexError("cross_entropy: target index out of range")
    return out.reshape(1, 1)


def cross_entropy_backward(logits, targets, g: float = 1.0):
    """backend.rs:2686-2712: (softmax(row) - onehot(target)) * g / rows."""
    l, t = _f32(logits), _f32(targets)
    out = np.empty_like(l)
    cols = l.shape[-1]
    if lib().oracle_cross_entropy_backward(_f(l), _f(t), t.size, l.size // cols, cols, g,
                                           _f(out)) != 0:
        raise IndexError("cross_entropy: target index out of range")
    return out


def mse(p, t):
    """backend.rs:2765-2772: mean of (p - t)^2."""
    p, t = _f32(p), _f32(t)
    return np.array([[lib().oracle_mse(_f(p), _f(t), p.size)]], np.float32)


def mse_backward(p, t, g: float = 1.0):
    """backend.rs:2780-2790: 2 * (p - t) * g / n."""
    p, t = _f32(p), _f32(t)
    out = np.empty_like(p)
    lib().oracle_mse_backward(_f(p), _f(t), p.size, g, _f(out))
    return out


def adamw(w, g, m, v, step: int, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8,
          weight_decay=0.01, loss_scale=65536.0, clip=1.0):
    """optim.rs:375-395: one AdamW step; returns updated copies (w, m, v).
    Defaults are AdamW::new's (optim.rs:226-240) and the clip of 1.0 the
    step uses."""
    w, m, v = (np.array(a, dtype=np.float32, copy=True) for a in (w, m, v))
    g = _f32(g)
    lib().oracle_adamw(_f(w), _f(g), _f(m), _f(v), w.size, lr, beta1, beta2, eps, weight_decay,
                       loss_scale, clip, step)
    return w, m, v


def rope(x, head_dim: int, pos_offset: int = 0):
    """backend.rs:2797-2826: x [B, S, hidden] or [S, hidden]."""
    x = _f32(x)
    b, s_ = (x.shape[0], x.shape[1]) if x.ndim == 3 else (1, x.shape[0])
    out = np.empty_like(x)
    lib().oracle_rope(_f(x), b, s_, x.shape[-1], head_dim, pos_offset, _f(out))
    return out


ATTN_CAUSAL, ATTN_ROPE = 1, 2


def attention(q, k, v, num_heads: int, q_pos: int = 0, k_pos: int = 0,
              flags: int = ATTN_CAUSAL | ATTN_ROPE, scale: Optional[float] = None,
              rows: Optional[tuple] = None):
    """The prefill attention lazy.rs:4821-4909 fuses, with an exact exp:
    q [B, S, H*D] (or [S, H*D]), k, v [B, Sk, H*D]; see clove_oracle.c.
    rows = (s_lo, s_hi) computes only those query rows (others are 0)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    two_d = q.ndim == 2
    if two_d:
        q, k, v = q[None], k[None], v[None]
    B, S, HD = q.shape
    Sk = k.shape[1]
    D = HD // num_heads
    sc = float(1.0 / np.sqrt(np.float32(D))) if scale is None else scale
    out = np.zeros_like(q)
    s_lo, s_hi = rows or (0, S)
    lib().oracle_attention(_f(q), _f(k), _f(v), B, S, Sk, num_heads, D, q_pos, k_pos, flags,
                           sc, s_lo, s_hi, _f(out))
    return out[0] if two_d else out
