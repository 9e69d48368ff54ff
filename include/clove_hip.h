/*
 * clove_hip.h -- C ABI of the MI355X (gfx950) backend for Clove's hot path.
 *
 * This is the drop-in boundary: a Rust `impl Backend for HipBackend` (or any
 * other FFI caller) binds these symbols the way Clove's own C bridge binds
 * `WgpuBackend` (reference src/ffi.rs).  Every entry takes plain pointers,
 * sizes and opaque handles; no C++ or torch types cross it.
 *
 * Conventions
 *   - A CTensor is an opaque handle to one device allocation (f32 or int32)
 *     plus its shape, mirroring ffi.rs:35 `pub type CTensor = *mut c_void`.
 *   - Ops return a NEW handle that the caller frees with clove_hip_tensor_free
 *     (ffi.rs:119-266).  On any error they return NULL and record a message
 *     for clove_hip_last_error(); functions returning int return 0 (CLOVE_HIP_OK)
 *     or a CLOVE_HIP_ERR_* code.  The reference aborts on errors (panic with
 *     panic = "abort", Cargo.toml:43); status codes replace that.
 *   - All device work is ordered on ONE HIP stream.  Ops only enqueue work;
 *     clove_hip_tensor_data / clove_hip_tensor_read / clove_hip_synchronize
 *     are the synchronisation points (the counterpart of to_cpu,
 *     backend.rs:1056-1090).
 *   - The API is thread-safe: one global lock orders host-side calls.
 */
#ifndef CLOVE_HIP_H
#define CLOVE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *CTensor;                       /* ffi.rs:35 */
typedef struct clove_hip_graph clove_hip_graph; /* lazy.rs:30-33 GLOBAL_GRAPH, made explicit */
typedef struct clove_hip_model clove_hip_model; /* lazy.rs:2545 CompiledModel */

enum clove_hip_status {
    CLOVE_HIP_OK = 0,
    CLOVE_HIP_ERR_INVALID = 1,   /* null handle / bad argument */
    CLOVE_HIP_ERR_SHAPE = 2,     /* shapes do not satisfy the op's rule */
    CLOVE_HIP_ERR_HIP = 3,       /* a HIP runtime call failed */
    CLOVE_HIP_ERR_JIT = 4,       /* runtime compilation of a fused chain failed */
    CLOVE_HIP_ERR_OOM = 5,       /* device allocation failed */
    CLOVE_HIP_ERR_NOT_INIT = 6,  /* clove_hip_init was not called */
    CLOVE_HIP_ERR_RANGE = 7      /* an index (block table, context length) is out of range */
};

enum clove_hip_dtype { CLOVE_HIP_F32 = 0, CLOVE_HIP_I32 = 1 };

/* Opcodes: the hot-path subset of Clove's IR (backend.rs:85-127), used by the
 * fused-chain entry and by the graph builder. */
enum clove_hip_opcode {
    CLOVE_OP_INPUT = 0,
    CLOVE_OP_MATMUL = 1,
    CLOVE_OP_ADD = 2,
    CLOVE_OP_SUB = 3,
    CLOVE_OP_MUL = 4,
    CLOVE_OP_SCALAR_MUL = 5,   /* param = factor */
    CLOVE_OP_FLATTEN = 6,      /* identity on data */
    CLOVE_OP_RELU = 7,
    CLOVE_OP_GELU = 8,
    CLOVE_OP_SIN = 9,
    CLOVE_OP_COS = 10,
    CLOVE_OP_SOFTMAX = 11,
    CLOVE_OP_LAYER_NORM = 12,  /* deps: x, gamma, beta */
    CLOVE_OP_DROPOUT = 13,     /* param = rate; fused form scales by 1/(1-rate), lazy.rs:1795-1803 */
    CLOVE_OP_RELU_GRAD = 14,   /* deps: x, grad_out */
    CLOVE_OP_GELU_GRAD = 15,   /* deps: x, grad_out */
    CLOVE_OP_CAST = 16,        /* identity on f32 data, lazy.rs:1808-1814 */
    CLOVE_OP_SIGMOID = 17,
    CLOVE_OP_TANH = 18,
    CLOVE_OP_PAGED_ATTENTION = 19, /* deps: q, k, v, kv_cache, block_tables, context_lens */
    CLOVE_OP_ROPE = 20         /* RoPE(pos_offset, head_dim), backend.rs:111; deps: x.
                                  Added with clove_hip_graph_rope (two integer parameters) */
};

/* ---------------------------------------------------------------------- */
/* Device lifecycle.  Replaces EngineDevice::init (device.rs:79-150).      */
/* ---------------------------------------------------------------------- */

int clove_hip_init(int device_ordinal);
int clove_hip_shutdown(void);
/* Message of the last failed call on this thread ("" when none). */
const char *clove_hip_last_error(void);
/* Status code of the last call on this thread (CLOVE_HIP_OK when it succeeded);
 * lets handle-returning entries report why they returned NULL. */
int clove_hip_last_status(void);
int clove_hip_synchronize(void);
/* Use a caller-owned hipStream_t (passed as void*) for all later work;
 * NULL restores the library's own stream.  Waits for the work already queued
 * on the stream it replaces. */
int clove_hip_set_stream(void *hip_stream);
void *clove_hip_get_stream(void);
/* Return cached free device blocks to the driver. */
int clove_hip_empty_cache(void);
/* Bytes currently held by the caching allocator (in use + cached). */
size_t clove_hip_memory_reserved(void);
/* Fused chains this process compiled with hipRTC, and chains it loaded from
 * the on-disk code-object cache (directory CLOVE_JIT_CACHE, default
 * $XDG_CACHE_HOME/clove_hip or $HOME/.cache/clove_hip; "0" turns it off).
 * No counterpart in the reference (its WGSL pipelines are rebuilt by wgpu
 * in every process); for callers that track start-up cost. */
int clove_hip_jit_stats(int *compiled, int *disk_loads);

/* ---------------------------------------------------------------------- */
/* Tensor lifecycle.  ffi.rs:71-113.                                      */
/* ---------------------------------------------------------------------- */

/* ffi.rs:71-87 clove_tensor_create(data, rows, cols): copies host data. */
CTensor clove_hip_tensor_create(const float *data, size_t rows, size_t cols);
/* N-d f32 / int32 tensors (block tables and context lengths are int32). */
CTensor clove_hip_tensor_create_nd(const float *data, const size_t *shape, size_t ndim);
CTensor clove_hip_tensor_create_i32(const int32_t *data, const size_t *shape, size_t ndim);
/* Uninitialised device tensor of the given dtype. */
CTensor clove_hip_tensor_empty(const size_t *shape, size_t ndim, int dtype);
/* Non-owning view of caller-owned device memory (freed by the caller). */
CTensor clove_hip_tensor_wrap(void *device_ptr, const size_t *shape, size_t ndim, int dtype);
/* ffi.rs:89-97 clove_tensor_free.  NULL is ignored. */
void clove_hip_tensor_free(CTensor t);
/* ffi.rs:99-113 clove_tensor_data: downloads all elements (f32 tensors). */
int clove_hip_tensor_data(CTensor t, float *out);
/* Element-range download / upload for either dtype (offset and count in elements). */
int clove_hip_tensor_read(CTensor t, void *out, size_t offset, size_t count);
int clove_hip_tensor_write(CTensor t, const void *src, size_t offset, size_t count);
size_t clove_hip_tensor_ndim(CTensor t);
int clove_hip_tensor_shape(CTensor t, size_t *shape_out);
size_t clove_hip_tensor_numel(CTensor t);
int clove_hip_tensor_dtype(CTensor t);
void *clove_hip_tensor_device_ptr(CTensor t);
/* Seeded synthetic data on the device (counter-based splitmix64 stream,
 * Box-Muller for normals).  Used to build benchmark-sized inputs without a
 * host round trip; tests download the bytes before comparing. */
int clove_hip_tensor_fill_normal(CTensor t, uint64_t seed, float mean, float stddev);
int clove_hip_tensor_fill_uniform(CTensor t, uint64_t seed, float lo, float hi);

/* ---------------------------------------------------------------------- */
/* Eager ops: the hot-path methods of `trait Backend` (backend.rs:171-257) */
/* as exported by ffi.rs.  Broadcast rule for add/sub/mul: b is read as    */
/* b[i % numel(b)] (backend.rs:1489, :1623, :1754).                        */
/* ---------------------------------------------------------------------- */

CTensor clove_hip_add(CTensor a, CTensor b);          /* ffi.rs:119-122, backend.rs:1483 */
CTensor clove_hip_sub(CTensor a, CTensor b);          /* ffi.rs:124-127, backend.rs:1748 */
CTensor clove_hip_mul(CTensor a, CTensor b);          /* ffi.rs:129-132, backend.rs:1598 */
CTensor clove_hip_mul_scalar(CTensor a, float s);     /* ffi.rs:139-142, backend.rs:1686 */
/* 2-d a [rows, cols] -> [cols, rows]; other ranks are CLOVE_HIP_ERR_SHAPE
 * (the reference reads shape[0] and shape[1] only). */
CTensor clove_hip_transpose(CTensor a);                 /* ffi.rs:144-147, backend.rs:2266 */
/* A copy of a with shape [1, numel(a)]. */
CTensor clove_hip_flatten(CTensor a);                   /* ffi.rs:149-152, backend.rs:2337 */
/* Per batch, a's rows then b's: [B, s1, h] + [B, s2, h] -> [B, s1 + s2, h]
 * (a 2-d operand is one batch; the result has a's rank).  Different batch or
 * hidden sizes are CLOVE_HIP_ERR_SHAPE. */
CTensor clove_hip_concat(CTensor a, CTensor b);         /* ffi.rs:154-157, backend.rs:1437 */
CTensor clove_hip_relu(CTensor a);                    /* ffi.rs:163-166, backend.rs:1815 */
CTensor clove_hip_gelu(CTensor a);                    /* ffi.rs:168-171, backend.rs:1917 */
CTensor clove_hip_sigmoid(CTensor a);                 /* ffi.rs:173-176, backend.rs:2951 */
CTensor clove_hip_tanh(CTensor a);                    /* ffi.rs:178-181, backend.rs:3008 */
CTensor clove_hip_sin(CTensor a);                     /* ffi.rs:188-191, backend.rs:1986 */
CTensor clove_hip_cos(CTensor a);                     /* ffi.rs:193-196, backend.rs:2044 */
/* Row softmax over the last dimension (backend.rs:2102-2125 uses
 * rows = shape[0], cols = shape[1]; identical for 2-d inputs). */
CTensor clove_hip_softmax(CTensor a);                 /* ffi.rs:183-186 */
/* Row layer norm over the last dimension, biased variance, eps 1e-5,
 * out = ((x-mean)/sqrt(var+eps))*gamma[j] + beta[j] (backend.rs:2380-2405). */
CTensor clove_hip_layer_norm(CTensor a, CTensor gamma, CTensor beta); /* ffi.rs:231-241 */
/* C = A.B with m = prod(a.shape[..last]), k = a.shape[last], n = b.shape[1]
 * (backend.rs:1282-1306); f32 accumulate on CDNA4 matrix cores. */
CTensor clove_hip_matmul(CTensor a, CTensor b);       /* ffi.rs:134-137 */

/* PagedAttention decode (backend.rs:249-256, ffi.rs:247-266).
 *   q            f32 [B, H*D] (any shape with numel B*H*D)
 *   k, v         f32 [B, H*D] freshly projected token, or NULL.  When given,
 *                token ctx_b-1 of sequence b is read from them instead of
 *                from the cache; when NULL every token comes from the cache.
 *   kv_cache     f32 [2, num_blocks, block_size, H, D]: plane 0 keys,
 *                plane 1 values (the per-plane layout of nn.rs:534)
 *   block_tables int32 [B, max_blocks] (nn.rs:535)
 *   context_lens int32 [B]
 * Returns out f32 with q's shape: out = softmax(q.K^T / sqrt(D)) V per
 * (sequence, head).  Any head_dim D in 1..1024 and any block_size >= 1
 * (head_dim = dim / num_heads is unrestricted in nn.rs:519); D 64/128/256
 * with block sizes 8/16/32 run a fixed-shape kernel, the rest a general one.
 * Fails with CLOVE_HIP_ERR_RANGE if a context length exceeds
 * max_blocks*block_size or a table entry used lies outside the pool. */
CTensor clove_hip_paged_attention(CTensor q, CTensor k, CTensor v, CTensor kv_cache,
                                  CTensor block_tables, CTensor context_lens);
/* Same with an explicit softmax scale (the reference uses 1/sqrt(D),
 * lazy.rs:5267). */
CTensor clove_hip_paged_attention_scaled(CTensor q, CTensor k, CTensor v, CTensor kv_cache,
                                         CTensor block_tables, CTensor context_lens,
                                         float scale);
/* Allocation-free paged decode.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Computes what
 * clove_hip_paged_attention_scaled computes, with the same kernels, on
 * caller-owned device memory given as plain pointers:
 *   q, out       f32 [num_seqs, num_heads*head_dim]
 *   k, v         f32 [num_seqs, num_heads*head_dim] new token, or both NULL
 *   kv_cache     f32 [2, num_blocks, block_size, num_heads, head_dim]
 *   block_tables int32 [num_seqs, max_blocks]; context_lens int32 [num_seqs]
 * all 16-byte aligned (4-byte when head_dim % 4 != 0); scale is used as given.  The partition workspace
 * (num_seqs*num_heads*partitions*(head_dim+2) floats when a context spans
 * more than one partition) lives in a static 16 MiB device array per GPU;
 * a shape needing more fails with CLOVE_HIP_ERR_SHAPE before any launch.
 * Nothing is allocated.  Calls made through this library never overlap:
 * every call runs on the library's current stream, and clove_hip_set_stream
 * waits for the stream it replaces.  Work that replays such a call outside
 * the library (a captured graph launched on two streams at once) shares the
 * array and races; the caller must order those replays.  Index errors are
 * reported as by the other paged entries. */
int clove_hip_paged_attention_noalloc(const float *q, const float *k, const float *v,
                                      const float *kv_cache, int64_t num_blocks, int block_size,
                                      int num_heads, int head_dim, const int32_t *block_tables,
                                      int max_blocks, const int32_t *context_lens, int num_seqs,
                                      float scale, float *out);
/* KV-cache append: writes each sequence's new-token k[b] and v[b] (f32
 * [B, H*D]) into planes 0 and 1 of kv_cache at the slot of token ctx_b - 1,
 * bt[b][(ctx_b-1)/bs]*bs + (ctx_b-1)%bs.  Sequences with ctx_b <= 0 are
 * skipped.  Afterwards paged_attention(q, NULL, NULL, ...) equals
 * paged_attention(q, k, v, ...) bit for bit.  Clove has no counterpart: this is
 * the cache write that must precede decode (the k/v projections of
 * nn.rs:540-542 never reach kv_cache in the reference).  Table entries outside
 * the pool are skipped and reported by the next synchronising call. */
int clove_hip_paged_kv_append(CTensor kv_cache, CTensor k, CTensor v, CTensor block_tables,
                              CTensor context_lens);
/* Gather-index debug entry: int32 [B, max_ctx] of physical token slots
 * bt[b][t/bs]*bs + t%bs (lazy.rs:5262-5270), -1 where t >= ctx_b.  Computed
 * on the device by the same index code the attention kernel uses. */
CTensor clove_hip_paged_gather_indices(CTensor block_tables, CTensor context_lens,
                                       int block_size, int max_ctx);

/* ---------------------------------------------------------------------- */
/* Backward passes and losses: the autograd closures WgpuBackend attaches  */
/* to its ops (backend.rs), as device ops returning new tensors.  Every    */
/* reduction sums in a fixed order (the reference's WGSL uses f32          */
/* compare-and-swap atomics), so results repeat bit for bit.               */
/* ---------------------------------------------------------------------- */

/* backend.rs:1858-1870 (relu backward): grad_out where x > 0, else 0 (x or
 * relu(x) may be passed: both are positive at the same places). */
CTensor clove_hip_relu_backward(CTensor x, CTensor grad_out);
/* backend.rs:1965-1981 (gelu backward): grad_out times the derivative of
 * the tanh-form GELU at x. */
CTensor clove_hip_gelu_backward(CTensor x, CTensor grad_out);
/* backend.rs:2163-2183 (softmax backward): from y = softmax(x) and
 * grad_out, per row dx = y * (grad_out - sum(grad_out * y)). */
CTensor clove_hip_softmax_backward(CTensor y, CTensor grad_out);
/* backend.rs:1314-1360 (matmul backward): *grad_a = grad_out . b^T (with
 * a's shape), *grad_b = a^T . grad_out ([k, n]); grad_out holds m*n
 * elements (m = product of a's leading dims).  Either output pointer may be
 * NULL to skip that product.  Returns a status. */
int clove_hip_matmul_backward(CTensor a, CTensor b, CTensor grad_out, CTensor *grad_a,
                              CTensor *grad_b);
/* backend.rs:1527-1538 (add) and 1800-1810 (sub): gradient of the
 * broadcast operand b, gb[i % b_numel] += grad_out[i] (negate = 0, add) or
 * -= (negate = 1, sub); f32 [b_numel].  (The reference's WGSL version folds
 * each workgroup into one bin through a CAS loop, backend.rs:596-645.) */
CTensor clove_hip_broadcast_grad(CTensor grad_out, size_t b_numel, int negate);
/* backend.rs:2661-2680 (cross entropy): logits f32 [rows, cols] (rows = all
 * leading dims), targets f32 class indices; the first min(rows,
 * numel(targets)) rows contribute -log softmax(row)[target] and the sum is
 * divided by rows.  Returns f32 [1, 1].  A class >= cols (a panic in the
 * reference) is reported as CLOVE_HIP_ERR_RANGE by the next synchronising
 * call. */
CTensor clove_hip_cross_entropy(CTensor logits, CTensor targets);
/* backend.rs:2686-2712: (softmax(row) - onehot(target)) * grad_loss / rows,
 * rows without a target get 0; grad_loss is a 1-element tensor. */
CTensor clove_hip_cross_entropy_backward(CTensor logits, CTensor targets, CTensor grad_loss);
/* backend.rs:2765-2772 (mse): mean over pred's elements of
 * (pred - target)^2; f32 [1, 1]. */
CTensor clove_hip_mse(CTensor pred, CTensor target);
/* backend.rs:2780-2790: 2 * (pred - target) * grad_loss / numel(pred). */
CTensor clove_hip_mse_backward(CTensor pred, CTensor target, CTensor grad_loss);

/* Attention prefill: the computation of the lazy path's fused FlashAttention
 * step (pattern MatMul(Softmax(MatMul(rope(q), rope(k)))), v), lazy.rs:
 * 1621-1690; kernel lazy.rs:4821-4909), with an exact exp (the reference
 * uses (1 + x/8)^8), batched and multi-head.  q f32 [B, S, H*D] or [S, H*D];
 * k, v f32 [B, Sk, H*D] (same rank as q).  num_heads = H; D = 64 or 128.
 * flags: CLOVE_ATTN_CAUSAL masks keys with t + k_pos > s + q_pos;
 * CLOVE_ATTN_ROPE rotates q and k at positions s + q_pos and t + k_pos as
 * clove_hip_rope does (the reference kernel always does both).  scale <= 0
 * selects 1/sqrt(D).  Returns out with q's shape; a query with no visible
 * key gets zeros. */
#define CLOVE_ATTN_CAUSAL 1
#define CLOVE_ATTN_ROPE 2
CTensor clove_hip_flash_attention(CTensor q, CTensor k, CTensor v, int num_heads, int q_pos,
                                  int k_pos, int flags, float scale);
/* backend.rs:221, 2797-2826 (rope): x f32 [B, S, hidden] or [S, hidden];
 * pair (i, i+1) of each head_dim-wide head at position s + pos_offset
 * rotates by theta = pos / 10000^(i / head_dim); dims past the last whole
 * head come out 0, as in the reference.  head_dim even, at most 256. */
CTensor clove_hip_rope(CTensor x, size_t pos_offset, size_t head_dim);

/* optim.rs:375-395 (AdamW::step, the Rayon branch; WGSL :305-345): one
 * fused AdamW update, in place on weights[i], m[i] and v[i] for i < count,
 * with grads[i] the gradients (f32, one element count per i).  Per element:
 * decoupled decay w -= lr*wd*w, g' = clamp(g / loss_scale, -clip, clip),
 * m = b1*m + (1-b1)*g', v = b2*v + (1-b2)*g'*g', and
 * w -= lr * (m / (1 - b1^t)) / (sqrt(v / (1 - b2^t)) + eps).  step is
 * AdamW's step_count after its increment (1 on the first step); m and v
 * start as zeros.  The reference uses beta1 0.9, beta2 0.999, eps 1e-8,
 * weight_decay 0.01, loss_scale 65536 and clip 1.0.  One launch covers up
 * to 16 tensors.  Returns a status. */
int clove_hip_adamw_step(CTensor *weights, CTensor *grads, CTensor *m, CTensor *v, int count,
                         float lr, float beta1, float beta2, float eps, float weight_decay,
                         float loss_scale, float clip, unsigned int step);

/* ---------------------------------------------------------------------- */
/* Fused elementwise chain: the counterpart of Step::Fused                 */
/* (codegen lazy.rs:1694-1838, broadcast rule lazy.rs:1600-1608).         */
/* ---------------------------------------------------------------------- */

typedef struct clove_hip_chain_op {
    int32_t opcode;  /* CLOVE_OP_ADD .. CLOVE_OP_TANH (elementwise subset) */
    int32_t src0;    /* operand: >= 0 earlier op of the chain, < 0 input -(src+1) */
    int32_t src1;    /* second operand for binary ops, ignored otherwise */
    int32_t store;   /* nonzero: materialise this op's value (last op always is) */
    float param;     /* SCALAR_MUL factor or DROPOUT rate */
} clove_hip_chain_op;

/* Evaluates the chain per element of the output index space (numel of the
 * last op = numel of its first operand chain), reading input k as
 * input_k[idx % numel(input_k)].  Writes one new tensor per op with `store`
 * set (and for the last op) into `outputs`, in op order; returns how many it
 * wrote, or a negative status on error.  Chains are compiled once per
 * structure with hipRTC for gfx950 and cached. */
int clove_hip_fused_chain(const clove_hip_chain_op *ops, int n_ops, const CTensor *inputs,
                          int n_inputs, CTensor *outputs);

/* ---------------------------------------------------------------------- */
/* Lazy graph: LazyBackend tracing (lazy.rs:36-1153), compile()           */
/* (lazy.rs:4273-5302) and CompiledModel::execute (lazy.rs:2545-4271).    */
/* ---------------------------------------------------------------------- */

clove_hip_graph *clove_hip_graph_create(void);
void clove_hip_graph_free(clove_hip_graph *g);
/* Adds an Input node.  `shape` is a comma-separated list of SymInt
 * expressions over integers and the symbols S0..S3 with + - * (for example
 * "S0,784" or "S0*16,128"), mirroring SymInt (backend.rs:30-69).  Returns the
 * node id or a negative status. */
int clove_hip_graph_input(clove_hip_graph *g, const char *shape);
/* Adds an op node over earlier node ids; the output shape follows the op's
 * rule.  Returns the node id or a negative status. */
int clove_hip_graph_op(clove_hip_graph *g, int opcode, const int *deps, int n_deps, float param);
/* Adds RoPE(pos_offset, head_dim) over node x: the LazyBackend trace of
 * rope (lazy.rs:475-480, Opcode::RoPE at backend.rs:111); x's shape.  On its
 * own it runs as clove_hip_rope does.  The planner fuses
 *   MatMul(Softmax(MatMul([ScalarMul(s)](RoPE(q, pq, D)), RoPE(k, pk, D))), v)
 * into one attention step (the FlashAttention pattern, lazy.rs:1621-1690,
 * with the contract of its kernel, lazy.rs:4821-4909): q [S, H*D] and k, v
 * [Sk, H*D] hold one token per row, H = hidden / D heads, q rotated at
 * s + pq and k at t + pk, keys t > s masked (on row indices, as the
 * reference kernel does), softmax scale s (1/sqrt(D) without a ScalarMul).
 * Returns the node id or a negative status. */
int clove_hip_graph_rope(clove_hip_graph *g, int x, size_t pos_offset, size_t head_dim);
/* Dead-code elimination, constant folding, fusion planning, liveness-based
 * buffer assignment and kernel compilation for the given outputs. */
clove_hip_model *clove_hip_compile(clove_hip_graph *g, const int *outputs, int n_outputs);
void clove_hip_model_free(clove_hip_model *m);
/* Inputs are bound in Input-node creation order; env holds S0..S3 (NULL
 * means all 1, as SymInt::eval defaults unknown symbols, backend.rs:43).
 * Writes one new tensor per requested output. */
int clove_hip_execute(clove_hip_model *m, const CTensor *inputs, int n_inputs,
                      const int64_t *env, CTensor *outputs);
/* Number of launched steps and a one-line-per-step description of the plan. */
int clove_hip_model_num_steps(clove_hip_model *m);
const char *clove_hip_model_describe(clove_hip_model *m);

/* ---------------------------------------------------------------------- */
/* Timing on the library's stream (for benchmarks).                        */
/* ---------------------------------------------------------------------- */

/* Records an event on the current stream; returns an id >= 0 or a negative status. */
int clove_hip_event_record(void);
/* Milliseconds between two recorded events (synchronises on the second). */
int clove_hip_event_elapsed(int ev_start, int ev_end, float *ms);
void clove_hip_event_reset(void);

#ifdef __cplusplus
}
#endif

#endif /* CLOVE_HIP_H */
