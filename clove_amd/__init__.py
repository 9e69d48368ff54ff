"""clove_amd -- Python binding of the MI355X HIP backend for Clove's hot path.

The product is the C-ABI library ``libclove_hip.so`` (include/clove_hip.h);
this module binds it with ctypes the way a foreign caller binds Clove's own C
bridge (reference src/ffi.rs), and adds a thin object layer:

* :class:`Tensor` owns one CTensor handle (ffi.rs:35-55); ``numpy()`` is the
  counterpart of ``clove_tensor_data`` (ffi.rs:99-113).
* The free functions mirror the hot-path methods of ``trait Backend``
  (backend.rs:171-257): ``add``, ``sub``, ``mul``, ``mul_scalar``, ``relu``,
  ``gelu``, ``sigmoid``, ``tanh``, ``sin``, ``cos``, ``softmax``,
  ``layer_norm``, ``matmul``, ``paged_attention``.
* :class:`Graph` mirrors LazyBackend tracing (lazy.rs:36-1153) and
  :meth:`Graph.compile` / :meth:`Model.execute` mirror ``compile`` and
  ``CompiledModel::execute`` (lazy.rs:4273, 2557).

There is no CPU fallback: importing works without a GPU, but every call that
needs the device fails with :class:`CloveError` unless ``init()`` succeeded on
a gfx950 device, and a missing library raises at load time.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Iterable, Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libclove_hip.so")

# Status codes (clove_hip.h)
OK = 0
ERR_INVALID, ERR_SHAPE, ERR_HIP, ERR_JIT, ERR_OOM, ERR_NOT_INIT, ERR_RANGE = 1, 2, 3, 4, 5, 6, 7
F32, I32 = 0, 1

# Opcodes (clove_hip.h, the hot-path subset of backend.rs:85-127)
OP = dict(
    INPUT=0, MATMUL=1, ADD=2, SUB=3, MUL=4, SCALAR_MUL=5, FLATTEN=6, RELU=7, GELU=8,
    SIN=9, COS=10, SOFTMAX=11, LAYER_NORM=12, DROPOUT=13, RELU_GRAD=14, GELU_GRAD=15,
    CAST=16, SIGMOID=17, TANH=18, PAGED_ATTENTION=19, ROPE=20,
)


class CloveError(RuntimeError):
    """A C-ABI call returned an error status (or NULL)."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[clove_hip error {code}] {msg}")
        self.code = code


class ChainOp(C.Structure):
    """clove_hip_chain_op: one op of a fused elementwise chain."""

    _fields_ = [("opcode", C.c_int32), ("src0", C.c_int32), ("src1", C.c_int32),
                ("store", C.c_int32), ("param", C.c_float)]


_lib: Optional[C.CDLL] = None


def _declare(lib: C.CDLL) -> None:
    vp, sz, i32p = C.c_void_p, C.c_size_t, C.POINTER(C.c_int32)
    szp = C.POINTER(C.c_size_t)
    f = C.c_float
    sig = {
        "clove_hip_init": (C.c_int, [C.c_int]),
        "clove_hip_shutdown": (C.c_int, []),
        "clove_hip_last_error": (C.c_char_p, []),
        "clove_hip_last_status": (C.c_int, []),
        "clove_hip_synchronize": (C.c_int, []),
        "clove_hip_jit_stats": (C.c_int, [C.POINTER(C.c_int), C.POINTER(C.c_int)]),
        "clove_hip_set_stream": (C.c_int, [vp]),
        "clove_hip_get_stream": (vp, []),
        "clove_hip_empty_cache": (C.c_int, []),
        "clove_hip_memory_reserved": (sz, []),
        "clove_hip_tensor_create": (vp, [C.POINTER(f), sz, sz]),
        "clove_hip_tensor_create_nd": (vp, [C.POINTER(f), szp, sz]),
        "clove_hip_tensor_create_i32": (vp, [i32p, szp, sz]),
        "clove_hip_tensor_empty": (vp, [szp, sz, C.c_int]),
        "clove_hip_tensor_wrap": (vp, [vp, szp, sz, C.c_int]),
        "clove_hip_tensor_free": (None, [vp]),
        "clove_hip_tensor_data": (C.c_int, [vp, C.POINTER(f)]),
        "clove_hip_tensor_read": (C.c_int, [vp, vp, sz, sz]),
        "clove_hip_tensor_write": (C.c_int, [vp, vp, sz, sz]),
        "clove_hip_tensor_ndim": (sz, [vp]),
        "clove_hip_tensor_shape": (C.c_int, [vp, szp]),
        "clove_hip_tensor_numel": (sz, [vp]),
        "clove_hip_tensor_dtype": (C.c_int, [vp]),
        "clove_hip_tensor_device_ptr": (vp, [vp]),
        "clove_hip_tensor_fill_normal": (C.c_int, [vp, C.c_uint64, f, f]),
        "clove_hip_tensor_fill_uniform": (C.c_int, [vp, C.c_uint64, f, f]),
        "clove_hip_add": (vp, [vp, vp]),
        "clove_hip_sub": (vp, [vp, vp]),
        "clove_hip_mul": (vp, [vp, vp]),
        "clove_hip_mul_scalar": (vp, [vp, f]),
        "clove_hip_transpose": (vp, [vp]),
        "clove_hip_flatten": (vp, [vp]),
        "clove_hip_concat": (vp, [vp, vp]),
        "clove_hip_relu": (vp, [vp]),
        "clove_hip_gelu": (vp, [vp]),
        "clove_hip_sigmoid": (vp, [vp]),
        "clove_hip_tanh": (vp, [vp]),
        "clove_hip_sin": (vp, [vp]),
        "clove_hip_cos": (vp, [vp]),
        "clove_hip_softmax": (vp, [vp]),
        "clove_hip_layer_norm": (vp, [vp, vp, vp]),
        "clove_hip_matmul": (vp, [vp, vp]),
        "clove_hip_paged_attention": (vp, [vp, vp, vp, vp, vp, vp]),
        "clove_hip_paged_attention_scaled": (vp, [vp, vp, vp, vp, vp, vp, f]),
        "clove_hip_paged_gather_indices": (vp, [vp, vp, C.c_int, C.c_int]),
        "clove_hip_paged_attention_noalloc": (C.c_int, [vp, vp, vp, vp, C.c_int64, C.c_int,
                                                        C.c_int, C.c_int, vp, C.c_int, vp,
                                                        C.c_int, f, vp]),
        "clove_hip_paged_kv_append": (C.c_int, [vp, vp, vp, vp, vp]),
        "clove_hip_relu_backward": (vp, [vp, vp]),
        "clove_hip_gelu_backward": (vp, [vp, vp]),
        "clove_hip_softmax_backward": (vp, [vp, vp]),
        "clove_hip_matmul_backward": (C.c_int, [vp, vp, vp, C.POINTER(vp), C.POINTER(vp)]),
        "clove_hip_broadcast_grad": (vp, [vp, sz, C.c_int]),
        "clove_hip_cross_entropy": (vp, [vp, vp]),
        "clove_hip_cross_entropy_backward": (vp, [vp, vp, vp]),
        "clove_hip_mse": (vp, [vp, vp]),
        "clove_hip_mse_backward": (vp, [vp, vp, vp]),
        "clove_hip_flash_attention": (vp, [vp, vp, vp, C.c_int, C.c_int, C.c_int, C.c_int, f]),
        "clove_hip_rope": (vp, [vp, sz, sz]),
        "clove_hip_adamw_step": (C.c_int, [C.POINTER(vp), C.POINTER(vp), C.POINTER(vp),
                                           C.POINTER(vp), C.c_int, f, f, f, f, f, f, f,
                                           C.c_uint]),
        "clove_hip_fused_chain": (C.c_int, [C.POINTER(ChainOp), C.c_int, C.POINTER(vp), C.c_int,
                                            C.POINTER(vp)]),
        "clove_hip_graph_create": (vp, []),
        "clove_hip_graph_free": (None, [vp]),
        "clove_hip_graph_input": (C.c_int, [vp, C.c_char_p]),
        "clove_hip_graph_op": (C.c_int, [vp, C.c_int, C.POINTER(C.c_int), C.c_int, f]),
        "clove_hip_graph_rope": (C.c_int, [vp, C.c_int, sz, sz]),
        "clove_hip_compile": (vp, [vp, C.POINTER(C.c_int), C.c_int]),
        "clove_hip_model_free": (None, [vp]),
        "clove_hip_execute": (C.c_int, [vp, C.POINTER(vp), C.c_int, C.POINTER(C.c_int64),
                                        C.POINTER(vp)]),
        "clove_hip_model_num_steps": (C.c_int, [vp]),
        "clove_hip_model_describe": (C.c_char_p, [vp]),
        "clove_hip_event_record": (C.c_int, []),
        "clove_hip_event_elapsed": (C.c_int, [C.c_int, C.c_int, C.POINTER(f)]),
        "clove_hip_event_reset": (None, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args


def lib() -> C.CDLL:
    """Loads libclove_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `make -C clove_amd/csrc` "
                "(or __graft_entry__.build()); there is no fallback implementation")
        handle = C.CDLL(LIB_PATH)
        _declare(handle)
        _lib = handle
    return _lib


def last_error() -> str:
    return lib().clove_hip_last_error().decode()


def _check(rc: int) -> None:
    if rc != OK:
        raise CloveError(rc, last_error())


def _handle(p) -> "Tensor":
    if not p:
        raise CloveError(lib().clove_hip_last_status(), last_error())
    return Tensor(p)


# ---------------------------------------------------------------------------
# device
# ---------------------------------------------------------------------------

def init(device: int = 0) -> None:
    """clove_hip_init: selects the device and creates the stream."""
    _check(lib().clove_hip_init(device))


def shutdown() -> None:
    _check(lib().clove_hip_shutdown())


def synchronize() -> None:
    _check(lib().clove_hip_synchronize())


def jit_stats() -> tuple:
    """(chains compiled with hipRTC, chains loaded from the on-disk
    code-object cache) in this process."""
    compiled, loaded = C.c_int(0), C.c_int(0)
    _check(lib().clove_hip_jit_stats(C.byref(compiled), C.byref(loaded)))
    return compiled.value, loaded.value


def empty_cache() -> None:
    _check(lib().clove_hip_empty_cache())


def memory_reserved() -> int:
    return int(lib().clove_hip_memory_reserved())


# ---------------------------------------------------------------------------
# tensors
# ---------------------------------------------------------------------------

def _shape_arr(shape: Sequence[int]):
    return (C.c_size_t * max(1, len(shape)))(*[int(s) for s in shape])


class Tensor:
    """Owns one CTensor handle; freed with clove_hip_tensor_free."""

    __slots__ = ("_h",)

    def __init__(self, handle):
        self._h = C.c_void_p(handle)

    @property
    def handle(self) -> C.c_void_p:
        return self._h

    def free(self) -> None:
        if self._h and self._h.value and _lib is not None:
            _lib.clove_hip_tensor_free(self._h)
        self._h = C.c_void_p(None)

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    @property
    def shape(self) -> tuple:
        nd = lib().clove_hip_tensor_ndim(self._h)
        arr = (C.c_size_t * max(1, nd))()
        _check(lib().clove_hip_tensor_shape(self._h, arr))
        return tuple(int(arr[i]) for i in range(nd))

    @property
    def numel(self) -> int:
        return int(lib().clove_hip_tensor_numel(self._h))

    @property
    def dtype(self):
        return np.float32 if lib().clove_hip_tensor_dtype(self._h) == F32 else np.int32

    @property
    def device_ptr(self) -> int:
        return int(lib().clove_hip_tensor_device_ptr(self._h) or 0)

    def numpy(self) -> np.ndarray:
        """Downloads the tensor (a synchronisation point)."""
        out = np.empty(self.shape, dtype=self.dtype)
        if out.size:
            _check(lib().clove_hip_tensor_read(self._h, out.ctypes.data_as(C.c_void_p), 0, out.size))
        else:
            synchronize()
        return out

    def read(self, offset: int, count: int) -> np.ndarray:
        out = np.empty(count, dtype=self.dtype)
        _check(lib().clove_hip_tensor_read(self._h, out.ctypes.data_as(C.c_void_p), offset, count))
        return out

    def write(self, offset: int, values: np.ndarray) -> None:
        v = np.ascontiguousarray(values, dtype=self.dtype).ravel()
        _check(lib().clove_hip_tensor_write(self._h, v.ctypes.data_as(C.c_void_p), offset, v.size))

    def fill_normal(self, seed: int, mean: float = 0.0, std: float = 1.0) -> "Tensor":
        _check(lib().clove_hip_tensor_fill_normal(self._h, seed, mean, std))
        return self

    def fill_uniform(self, seed: int, lo: float = 0.0, hi: float = 1.0) -> "Tensor":
        _check(lib().clove_hip_tensor_fill_uniform(self._h, seed, lo, hi))
        return self


def tensor(data, dtype=None) -> Tensor:
    """Uploads a numpy array (f32, or int32 for block tables / lengths)."""
    a = np.asarray(data)
    if dtype is None:
        dtype = np.int32 if a.dtype.kind in "iu" else np.float32
    a = np.ascontiguousarray(a, dtype=dtype)
    shape = a.shape if a.ndim else (1,)
    if dtype == np.int32:
        p = lib().clove_hip_tensor_create_i32(a.ctypes.data_as(C.POINTER(C.c_int32)),
                                              _shape_arr(shape), len(shape))
    else:
        p = lib().clove_hip_tensor_create_nd(a.ctypes.data_as(C.POINTER(C.c_float)),
                                             _shape_arr(shape), len(shape))
    return _handle(p)


def wrap(device_ptr: int, shape, dtype=np.float32) -> Tensor:
    """Borrows device memory the caller owns (clove_hip_tensor_wrap); the
    memory must outlive the handle, and freeing the handle leaves it alone."""
    code = 1 if dtype == np.int32 else 0
    return _handle(lib().clove_hip_tensor_wrap(C.c_void_p(device_ptr), _shape_arr(shape),
                                               len(shape), code))


def tensor2d(data) -> Tensor:
    """clove_hip_tensor_create(data, rows, cols), the 2-d form of ffi.rs:72."""
    a = np.ascontiguousarray(data, dtype=np.float32)
    assert a.ndim == 2
    return _handle(lib().clove_hip_tensor_create(a.ctypes.data_as(C.POINTER(C.c_float)),
                                                 a.shape[0], a.shape[1]))


def empty(shape: Sequence[int], dtype=np.float32) -> Tensor:
    return _handle(lib().clove_hip_tensor_empty(_shape_arr(shape), len(shape),
                                                I32 if dtype == np.int32 else F32))


# ---------------------------------------------------------------------------
# eager ops (trait Backend)
# ---------------------------------------------------------------------------

def add(a: Tensor, b: Tensor) -> Tensor:
    return _handle(lib().clove_hip_add(a.handle, b.handle))


def sub(a: Tensor, b: Tensor) -> Tensor:
    return _handle(lib().clove_hip_sub(a.handle, b.handle))


def mul(a: Tensor, b: Tensor) -> Tensor:
    return _handle(lib().clove_hip_mul(a.handle, b.handle))


def mul_scalar(a: Tensor, s: float) -> Tensor:
    return _handle(lib().clove_hip_mul_scalar(a.handle, s))


def transpose(a: Tensor) -> Tensor:
    """2-d [rows, cols] -> [cols, rows] (backend.rs:2266)."""
    return _handle(lib().clove_hip_transpose(a.handle))


def flatten(a: Tensor) -> Tensor:
    """A copy with shape [1, numel] (backend.rs:2337)."""
    return _handle(lib().clove_hip_flatten(a.handle))


def concat_seq(a: Tensor, b: Tensor) -> Tensor:
    """Per batch, a's rows then b's (backend.rs:1437)."""
    return _handle(lib().clove_hip_concat(a.handle, b.handle))


def relu(a: Tensor) -> Tensor:
    return _handle(lib().clove_hip_relu(a.handle))


def gelu(a: Tensor) -> Tensor:
    return _handle(lib().clove_hip_gelu(a.handle))


def sigmoid(a: Tensor) -> Tensor:
    return _handle(lib().clove_hip_sigmoid(a.handle))


def tanh(a: Tensor) -> Tensor:
    return _handle(lib().clove_hip_tanh(a.handle))


def sin(a: Tensor) -> Tensor:
    return _handle(lib().clove_hip_sin(a.handle))


def cos(a: Tensor) -> Tensor:
    return _handle(lib().clove_hip_cos(a.handle))


def softmax(a: Tensor) -> Tensor:
    return _handle(lib().clove_hip_softmax(a.handle))


def layer_norm(a: Tensor, gamma: Tensor, beta: Tensor) -> Tensor:
    return _handle(lib().clove_hip_layer_norm(a.handle, gamma.handle, beta.handle))


def matmul(a: Tensor, b: Tensor) -> Tensor:
    return _handle(lib().clove_hip_matmul(a.handle, b.handle))


# ---- backward passes and losses (backend.rs autograd closures) -------------

def relu_backward(x: Tensor, grad_out: Tensor) -> Tensor:
    return _handle(lib().clove_hip_relu_backward(x.handle, grad_out.handle))


def gelu_backward(x: Tensor, grad_out: Tensor) -> Tensor:
    return _handle(lib().clove_hip_gelu_backward(x.handle, grad_out.handle))


def softmax_backward(y: Tensor, grad_out: Tensor) -> Tensor:
    """dx = y * (grad_out - sum(grad_out * y)) per row, y = softmax(x)."""
    return _handle(lib().clove_hip_softmax_backward(y.handle, grad_out.handle))


def matmul_backward(a: Tensor, b: Tensor, grad_out: Tensor, want_a: bool = True,
                    want_b: bool = True):
    """(grad_out . b^T, a^T . grad_out); a skipped product is None."""
    da, db = C.c_void_p(), C.c_void_p()
    _check(lib().clove_hip_matmul_backward(a.handle, b.handle, grad_out.handle,
                                           C.byref(da) if want_a else None,
                                           C.byref(db) if want_b else None))
    return (Tensor(da.value) if want_a else None), (Tensor(db.value) if want_b else None)


def broadcast_grad(grad_out: Tensor, b_numel: int, negate: bool = False) -> Tensor:
    """Gradient of add's (negate=False) or sub's (True) broadcast operand."""
    return _handle(lib().clove_hip_broadcast_grad(grad_out.handle, b_numel, int(negate)))


def cross_entropy(logits: Tensor, targets: Tensor) -> Tensor:
    return _handle(lib().clove_hip_cross_entropy(logits.handle, targets.handle))


def cross_entropy_backward(logits: Tensor, targets: Tensor, grad_loss: Tensor) -> Tensor:
    return _handle(lib().clove_hip_cross_entropy_backward(logits.handle, targets.handle,
                                                          grad_loss.handle))


def mse(pred: Tensor, target: Tensor) -> Tensor:
    return _handle(lib().clove_hip_mse(pred.handle, target.handle))


def mse_backward(pred: Tensor, target: Tensor, grad_loss: Tensor) -> Tensor:
    return _handle(lib().clove_hip_mse_backward(pred.handle, target.handle, grad_loss.handle))


ATTN_CAUSAL, ATTN_ROPE = 1, 2


def flash_attention(q: Tensor, k: Tensor, v: Tensor, num_heads: int, q_pos: int = 0,
                    k_pos: int = 0, flags: int = ATTN_CAUSAL | ATTN_ROPE,
                    scale: float = 0.0) -> Tensor:
    """Attention prefill (the fused FlashAttention step); scale 0 = 1/sqrt(D)."""
    return _handle(lib().clove_hip_flash_attention(q.handle, k.handle, v.handle, num_heads,
                                                   q_pos, k_pos, flags, scale))


def rope(x: Tensor, head_dim: int, pos_offset: int = 0) -> Tensor:
    return _handle(lib().clove_hip_rope(x.handle, pos_offset, head_dim))


def adamw_step(weights, grads, m, v, step: int, lr: float = 1e-3, beta1: float = 0.9,
               beta2: float = 0.999, eps: float = 1e-8, weight_decay: float = 0.01,
               loss_scale: float = 65536.0, clip: float = 1.0) -> None:
    """One fused AdamW update in place on lists of weights / moments
    (defaults: AdamW::new, optim.rs:226-240, and the step's clip of 1.0)."""
    n = len(weights)
    arr = lambda ts: (C.c_void_p * max(n, 1))(*[t.handle.value for t in ts])
    _check(lib().clove_hip_adamw_step(arr(weights), arr(grads), arr(m), arr(v), n, lr, beta1,
                                      beta2, eps, weight_decay, loss_scale, clip, step))


def paged_attention(q: Tensor, k: Optional[Tensor], v: Optional[Tensor], kv_cache: Tensor,
                    block_tables: Tensor, context_lens: Tensor,
                    scale: Optional[float] = None) -> Tensor:
    kh = k.handle if k is not None else None
    vh = v.handle if v is not None else None
    if scale is None:
        p = lib().clove_hip_paged_attention(q.handle, kh, vh, kv_cache.handle,
                                            block_tables.handle, context_lens.handle)
    else:
        p = lib().clove_hip_paged_attention_scaled(q.handle, kh, vh, kv_cache.handle,
                                                   block_tables.handle, context_lens.handle, scale)
    return _handle(p)


def paged_kv_append(kv_cache: Tensor, k: Tensor, v: Tensor, block_tables: Tensor,
                    context_lens: Tensor) -> None:
    """Writes each sequence's new-token k/v into its cache slot ctx-1."""
    _check(lib().clove_hip_paged_kv_append(kv_cache.handle, k.handle, v.handle,
                                           block_tables.handle, context_lens.handle))


def paged_gather_indices(block_tables: Tensor, context_lens: Tensor, block_size: int,
                         max_ctx: int) -> Tensor:
    return _handle(lib().clove_hip_paged_gather_indices(block_tables.handle, context_lens.handle,
                                                        block_size, max_ctx))


class FusedChain:
    """A fused elementwise chain bound to its inputs (Step::Fused,
    lazy.rs:1694-1838).  ``ops`` holds tuples ``(opname, src0, src1, store,
    param)``; operand ``>= 0`` names an earlier op, ``< 0`` names input
    ``-(src+1)``.  Calling it runs the chain and returns the stored values
    (the last op always) in op order.  The argument arrays are built once,
    so repeated calls cost one C call each."""

    def __init__(self, ops: Sequence[tuple], inputs: Sequence[Tensor]):
        self._n_ops = len(ops)
        self._ops = (ChainOp * len(ops))()
        for i, op in enumerate(ops):
            name, s0, s1, store, param = (tuple(op) + (0, 0, 0, 0.0))[:5]
            self._ops[i] = ChainOp(OP[name.upper()], s0, s1, 1 if store else 0, float(param))
        self._inputs = list(inputs)  # keeps the handles alive
        self._n_in = len(inputs)
        self._ins = (C.c_void_p * len(inputs))(*[t.handle.value for t in inputs])
        self._outs = (C.c_void_p * len(ops))()
        self._fn = lib().clove_hip_fused_chain

    def __call__(self) -> list:
        n = self._fn(self._ops, self._n_ops, self._ins, self._n_in, self._outs)
        if n < 0:
            raise CloveError(-n, last_error())
        return [Tensor(self._outs[i]) for i in range(n)]


def fused_chain(ops: Sequence[tuple], inputs: Sequence[Tensor]) -> list:
    """Runs one fused elementwise chain once; see :class:`FusedChain`."""
    return FusedChain(ops, inputs)()


# ---------------------------------------------------------------------------
# lazy graph
# ---------------------------------------------------------------------------

class Model:
    """A compiled plan (CompiledModel, lazy.rs:2545)."""

    def __init__(self, handle, n_outputs: int):
        self._h = C.c_void_p(handle)
        self.n_outputs = n_outputs

    def __del__(self):
        try:
            if self._h and self._h.value and _lib is not None:
                _lib.clove_hip_model_free(self._h)
        except Exception:
            pass

    @property
    def num_steps(self) -> int:
        return lib().clove_hip_model_num_steps(self._h)

    def describe(self) -> str:
        return lib().clove_hip_model_describe(self._h).decode()

    def execute(self, inputs: Sequence[Tensor], env: Optional[Sequence[int]] = None) -> list:
        ins = (C.c_void_p * max(1, len(inputs)))(*[t.handle.value for t in inputs])
        envp = None
        if env is not None:
            e = list(env) + [1] * (4 - len(env))
            envp = (C.c_int64 * 4)(*e[:4])
        outs = (C.c_void_p * self.n_outputs)()
        _check(lib().clove_hip_execute(self._h, ins, len(inputs), envp, outs))
        return [Tensor(outs[i]) for i in range(self.n_outputs)]


class Graph:
    """Explicit LazyBackend trace (lazy.rs:30-33 keeps it thread-local)."""

    def __init__(self):
        self._h = C.c_void_p(lib().clove_hip_graph_create())

    def __del__(self):
        try:
            if self._h and self._h.value and _lib is not None:
                _lib.clove_hip_graph_free(self._h)
        except Exception:
            pass

    def input(self, shape) -> int:
        spec = shape if isinstance(shape, str) else ",".join(str(s) for s in shape)
        rc = lib().clove_hip_graph_input(self._h, spec.encode())
        if rc < 0:
            raise CloveError(-rc, last_error())
        return rc

    def op(self, name: str, *deps: int, param: float = 0.0) -> int:
        arr = (C.c_int * max(1, len(deps)))(*deps)
        rc = lib().clove_hip_graph_op(self._h, OP[name.upper()], arr, len(deps), param)
        if rc < 0:
            raise CloveError(-rc, last_error())
        return rc

    def rope(self, x: int, head_dim: int, pos_offset: int = 0) -> int:
        """RoPE(pos_offset, head_dim) over node x (lazy.rs:475-480)."""
        rc = lib().clove_hip_graph_rope(self._h, x, pos_offset, head_dim)
        if rc < 0:
            raise CloveError(-rc, last_error())
        return rc

    def compile(self, outputs: Iterable[int]) -> Model:
        outs = list(outputs)
        arr = (C.c_int * len(outs))(*outs)
        p = lib().clove_hip_compile(self._h, arr, len(outs))
        if not p:
            raise CloveError(ERR_INVALID, last_error())
        return Model(p, len(outs))


# ---------------------------------------------------------------------------
# timing
# ---------------------------------------------------------------------------

def event_record() -> int:
    rc = lib().clove_hip_event_record()
    if rc < 0:
        raise CloveError(-rc, last_error())
    return rc


def event_elapsed(a: int, b: int) -> float:
    ms = C.c_float()
    _check(lib().clove_hip_event_elapsed(a, b, C.byref(ms)))
    return float(ms.value)


def event_reset() -> None:
    lib().clove_hip_event_reset()
