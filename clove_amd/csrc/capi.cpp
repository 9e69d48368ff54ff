// capi.cpp -- the extern "C" boundary declared in include/clove_hip.h.
//
// Handles follow Clove's C bridge (ffi.rs:35-55): a CTensor is a heap cell
// holding a shared TensorNode, created by every op and released by
// clove_hip_tensor_free.  Each entry takes the global API lock, converts
// library errors into a status code / NULL plus a thread-local message, and
// lets nothing escape (the reference panics and aborts instead).
#include <cmath>
#include <cstring>
#include <new>

#include "common.hpp"
#include "graph.hpp"
#include "runtime.hpp"

using clove::Error;
using clove::Tensor;
using clove::TensorNode;

struct clove_hip_graph {
    clove::Graph g;
};
struct clove_hip_model {
    std::unique_ptr<clove::Model> m;
    std::string description;
};

namespace {

thread_local int g_last_status = CLOVE_HIP_OK;

CTensor into_raw(TensorNode t) { return new TensorNode(std::move(t)); }

TensorNode as_node(CTensor p) {
    if (!p) return nullptr;
    return *static_cast<TensorNode *>(p);
}

const Tensor &deref(CTensor p, const char *what) {
    if (!p) clove::fail(CLOVE_HIP_ERR_INVALID, std::string(what) + " is NULL");
    const TensorNode &n = *static_cast<TensorNode *>(p);
    if (!n) clove::fail(CLOVE_HIP_ERR_INVALID, std::string(what) + " is an empty handle");
    return *n;
}

std::vector<size_t> shape_of(const size_t *shape, size_t ndim) {
    if (!shape && ndim) clove::fail(CLOVE_HIP_ERR_INVALID, "shape is NULL");
    return std::vector<size_t>(shape, shape + ndim);
}

// Runs `f`, mapping errors to a status code.
template <class F>
int guarded(F &&f) {
    std::lock_guard<std::recursive_mutex> lk(clove::api_mutex());
    try {
        f();
        clove::set_last_error("");
        return g_last_status = CLOVE_HIP_OK;
    } catch (const Error &e) {
        clove::set_last_error(e.msg);
        return g_last_status = e.code;
    } catch (const std::bad_alloc &) {
        clove::set_last_error("host allocation failed");
        return g_last_status = CLOVE_HIP_ERR_OOM;
    } catch (const std::exception &e) {
        clove::set_last_error(e.what());
        return g_last_status = CLOVE_HIP_ERR_INVALID;
    }
}

// Runs `f` returning a tensor; NULL on error.
template <class F>
CTensor guarded_tensor(F &&f) {
    CTensor out = nullptr;
    guarded([&] { out = into_raw(f()); });
    return out;
}

}  // namespace

extern "C" {

int clove_hip_init(int device_ordinal) { return guarded([&] { clove::init(device_ordinal); }); }
int clove_hip_shutdown(void) { return guarded([] { clove::shutdown(); }); }
const char *clove_hip_last_error(void) { return clove::last_error().c_str(); }
int clove_hip_last_status(void) { return g_last_status; }
int clove_hip_synchronize(void) { return guarded([] { clove::synchronize(); }); }
int clove_hip_set_stream(void *s) { return guarded([&] { clove::set_stream(s); }); }
void *clove_hip_get_stream(void) {
    void *s = nullptr;
    guarded([&] { s = clove::ctx().stream; });
    return s;
}
int clove_hip_jit_stats(int *compiled, int *disk_loads) {
    return guarded([&] { clove::jit_stats(compiled, disk_loads); });
}
int clove_hip_empty_cache(void) {
    return guarded([] {
        clove::ctx();
        clove::dev_empty_cache();
    });
}
size_t clove_hip_memory_reserved(void) {
    size_t n = 0;
    guarded([&] { n = clove::dev_reserved(); });
    return n;
}

// ---- tensors -----------------------------------------------------------------

CTensor clove_hip_tensor_create(const float *data, size_t rows, size_t cols) {
    if (!data) {  // ffi.rs:78-80: a NULL data pointer returns NULL
        clove::set_last_error("data is NULL");
        g_last_status = CLOVE_HIP_ERR_INVALID;
        return nullptr;
    }
    return guarded_tensor([&] { return clove::HipBackend::new_cpu(data, {rows, cols}); });
}

CTensor clove_hip_tensor_create_nd(const float *data, const size_t *shape, size_t ndim) {
    return guarded_tensor([&] {
        if (!data) clove::fail(CLOVE_HIP_ERR_INVALID, "data is NULL");
        return clove::HipBackend::new_cpu(data, shape_of(shape, ndim));
    });
}

CTensor clove_hip_tensor_create_i32(const int32_t *data, const size_t *shape, size_t ndim) {
    return guarded_tensor([&] {
        if (!data) clove::fail(CLOVE_HIP_ERR_INVALID, "data is NULL");
        TensorNode t = clove::new_tensor(shape_of(shape, ndim), CLOVE_HIP_I32);
        clove::upload(*t, data, 0, t->numel);
        return t;
    });
}

CTensor clove_hip_tensor_empty(const size_t *shape, size_t ndim, int dtype) {
    return guarded_tensor([&] { return clove::new_tensor(shape_of(shape, ndim), dtype); });
}

CTensor clove_hip_tensor_wrap(void *device_ptr, const size_t *shape, size_t ndim, int dtype) {
    return guarded_tensor([&] {
        clove::ctx();
        if (!device_ptr) clove::fail(CLOVE_HIP_ERR_INVALID, "device_ptr is NULL");
        if (dtype != CLOVE_HIP_F32 && dtype != CLOVE_HIP_I32)
            clove::fail(CLOVE_HIP_ERR_INVALID, "unknown dtype");
        auto t = std::make_shared<Tensor>();
        t->data = device_ptr;
        t->shape = shape_of(shape, ndim);
        t->dtype = dtype;
        t->numel = clove::numel_of(t->shape);
        t->bytes = t->numel * 4;
        t->owned = false;
        return t;
    });
}

void clove_hip_tensor_free(CTensor t) {
    if (!t) return;
    std::lock_guard<std::recursive_mutex> lk(clove::api_mutex());
    delete static_cast<TensorNode *>(t);
}

int clove_hip_tensor_data(CTensor t, float *out) {
    return guarded([&] {
        const Tensor &x = deref(t, "tensor");
        if (!out) clove::fail(CLOVE_HIP_ERR_INVALID, "out is NULL");
        clove::download(x, out, 0, x.numel);
    });
}

int clove_hip_tensor_read(CTensor t, void *out, size_t offset, size_t count) {
    return guarded([&] {
        const Tensor &x = deref(t, "tensor");
        if (!out && count) clove::fail(CLOVE_HIP_ERR_INVALID, "out is NULL");
        clove::download(x, out, offset, count);
    });
}

int clove_hip_tensor_write(CTensor t, const void *src, size_t offset, size_t count) {
    return guarded([&] {
        const Tensor &x = deref(t, "tensor");
        if (!src && count) clove::fail(CLOVE_HIP_ERR_INVALID, "src is NULL");
        clove::upload(const_cast<Tensor &>(x), src, offset, count);
    });
}

size_t clove_hip_tensor_ndim(CTensor t) {
    size_t n = 0;
    guarded([&] { n = deref(t, "tensor").shape.size(); });
    return n;
}

int clove_hip_tensor_shape(CTensor t, size_t *shape_out) {
    return guarded([&] {
        const Tensor &x = deref(t, "tensor");
        if (!shape_out && !x.shape.empty()) clove::fail(CLOVE_HIP_ERR_INVALID, "shape_out is NULL");
        std::copy(x.shape.begin(), x.shape.end(), shape_out);
    });
}

size_t clove_hip_tensor_numel(CTensor t) {
    size_t n = 0;
    guarded([&] { n = deref(t, "tensor").numel; });
    return n;
}

int clove_hip_tensor_dtype(CTensor t) {
    int d = -1;
    guarded([&] { d = deref(t, "tensor").dtype; });
    return d;
}

void *clove_hip_tensor_device_ptr(CTensor t) {
    void *p = nullptr;
    guarded([&] { p = deref(t, "tensor").data; });
    return p;
}

int clove_hip_tensor_fill_normal(CTensor t, uint64_t seed, float mean, float stddev) {
    return guarded([&] {
        clove::fill_normal(const_cast<Tensor &>(deref(t, "tensor")), seed, mean, stddev);
    });
}

int clove_hip_tensor_fill_uniform(CTensor t, uint64_t seed, float lo, float hi) {
    return guarded([&] {
        clove::fill_uniform(const_cast<Tensor &>(deref(t, "tensor")), seed, lo, hi);
    });
}

// ---- eager ops -----------------------------------------------------------------

using clove::HipBackend;

#define CLOVE_BINARY(name)                                                              \
    CTensor clove_hip_##name(CTensor a, CTensor b) {                                    \
        return guarded_tensor([&] {                                                     \
            deref(a, "a");                                                              \
            deref(b, "b");                                                              \
            return HipBackend::name(as_node(a), as_node(b));                            \
        });                                                                             \
    }
#define CLOVE_UNARY(name)                                                               \
    CTensor clove_hip_##name(CTensor a) {                                               \
        return guarded_tensor([&] {                                                     \
            deref(a, "a");                                                              \
            return HipBackend::name(as_node(a));                                        \
        });                                                                             \
    }

CLOVE_BINARY(add)
CLOVE_BINARY(sub)
CLOVE_BINARY(mul)
CLOVE_BINARY(matmul)
CLOVE_UNARY(relu)
CLOVE_UNARY(gelu)
CLOVE_UNARY(sigmoid)
CLOVE_UNARY(tanh)
CLOVE_UNARY(sin)
CLOVE_UNARY(cos)
CLOVE_UNARY(softmax)

CTensor clove_hip_mul_scalar(CTensor a, float s) {
    return guarded_tensor([&] {
        deref(a, "a");
        return HipBackend::mul_scalar(as_node(a), s);
    });
}

CTensor clove_hip_transpose(CTensor a) {
    return guarded_tensor([&] {
        deref(a, "a");
        return HipBackend::transpose(as_node(a));
    });
}

CTensor clove_hip_flatten(CTensor a) {
    return guarded_tensor([&] {
        deref(a, "a");
        return HipBackend::flatten(as_node(a));
    });
}

CTensor clove_hip_concat(CTensor a, CTensor b) {
    return guarded_tensor([&] {
        deref(a, "a");
        deref(b, "b");
        return HipBackend::concat_seq(as_node(a), as_node(b));
    });
}

CTensor clove_hip_layer_norm(CTensor a, CTensor gamma, CTensor beta) {
    return guarded_tensor([&] {
        deref(a, "a");
        deref(gamma, "gamma");
        deref(beta, "beta");
        return HipBackend::layer_norm(as_node(a), as_node(gamma), as_node(beta));
    });
}

CTensor clove_hip_paged_attention_scaled(CTensor q, CTensor k, CTensor v, CTensor kv_cache,
                                         CTensor block_tables, CTensor context_lens, float scale) {
    return guarded_tensor([&] {
        deref(q, "q");
        deref(kv_cache, "kv_cache");
        deref(block_tables, "block_tables");
        deref(context_lens, "context_lens");
        return HipBackend::paged_attention(as_node(q), as_node(k), as_node(v), as_node(kv_cache),
                                           as_node(block_tables), as_node(context_lens), scale);
    });
}

int clove_hip_paged_attention_noalloc(const float *q, const float *k, const float *v,
                                      const float *kv_cache, int64_t num_blocks, int block_size,
                                      int num_heads, int head_dim, const int32_t *block_tables,
                                      int max_blocks, const int32_t *context_lens, int num_seqs,
                                      float scale, float *out) {
    return guarded([&] {
        HipBackend::paged_attention_noalloc({q, k, v, kv_cache, num_blocks, block_size, num_heads,
                                             head_dim, block_tables, max_blocks, context_lens,
                                             num_seqs, scale, out});
    });
}

CTensor clove_hip_paged_attention(CTensor q, CTensor k, CTensor v, CTensor kv_cache,
                                  CTensor block_tables, CTensor context_lens) {
    return guarded_tensor([&] {
        const Tensor &kv = deref(kv_cache, "kv_cache");
        deref(q, "q");
        deref(block_tables, "block_tables");
        deref(context_lens, "context_lens");
        const float D = kv.shape.empty() ? 1.0f : (float)kv.shape.back();
        // lazy.rs:5267: scale = 1 / sqrt(head_dim)
        return HipBackend::paged_attention(as_node(q), as_node(k), as_node(v), as_node(kv_cache),
                                           as_node(block_tables), as_node(context_lens),
                                           1.0f / std::sqrt(D));
    });
}

int clove_hip_paged_kv_append(CTensor kv_cache, CTensor k, CTensor v, CTensor block_tables,
                              CTensor context_lens) {
    return guarded([&] {
        HipBackend::paged_kv_append(deref(kv_cache, "kv_cache"), deref(k, "k"), deref(v, "v"),
                                    deref(block_tables, "block_tables"),
                                    deref(context_lens, "context_lens"));
    });
}

// ---- backward passes and losses ------------------------------------------

CTensor clove_hip_relu_backward(CTensor x, CTensor grad_out) {
    return guarded_tensor([&] { return HipBackend::relu_backward(as_node(x), as_node(grad_out)); });
}

CTensor clove_hip_gelu_backward(CTensor x, CTensor grad_out) {
    return guarded_tensor([&] { return HipBackend::gelu_backward(as_node(x), as_node(grad_out)); });
}

CTensor clove_hip_softmax_backward(CTensor y, CTensor grad_out) {
    return guarded_tensor(
        [&] { return HipBackend::softmax_backward(as_node(y), as_node(grad_out)); });
}

int clove_hip_matmul_backward(CTensor a, CTensor b, CTensor grad_out, CTensor *grad_a,
                              CTensor *grad_b) {
    if (grad_a) *grad_a = nullptr;
    if (grad_b) *grad_b = nullptr;
    TensorNode da, db;
    const int st = guarded([&] {
        HipBackend::matmul_backward(as_node(a), as_node(b), as_node(grad_out),
                                    grad_a ? &da : nullptr, grad_b ? &db : nullptr);
    });
    if (st == CLOVE_HIP_OK) {
        if (grad_a) *grad_a = into_raw(std::move(da));
        if (grad_b) *grad_b = into_raw(std::move(db));
    }
    return st;
}

CTensor clove_hip_broadcast_grad(CTensor grad_out, size_t b_numel, int negate) {
    return guarded_tensor(
        [&] { return HipBackend::broadcast_grad(as_node(grad_out), b_numel, negate != 0); });
}

CTensor clove_hip_cross_entropy(CTensor logits, CTensor targets) {
    return guarded_tensor(
        [&] { return HipBackend::cross_entropy(as_node(logits), as_node(targets)); });
}

CTensor clove_hip_cross_entropy_backward(CTensor logits, CTensor targets, CTensor grad_loss) {
    return guarded_tensor([&] {
        return HipBackend::cross_entropy_backward(as_node(logits), as_node(targets),
                                                  as_node(grad_loss));
    });
}

CTensor clove_hip_mse(CTensor pred, CTensor target) {
    return guarded_tensor([&] { return HipBackend::mse(as_node(pred), as_node(target)); });
}

CTensor clove_hip_mse_backward(CTensor pred, CTensor target, CTensor grad_loss) {
    return guarded_tensor([&] {
        return HipBackend::mse_backward(as_node(pred), as_node(target), as_node(grad_loss));
    });
}

CTensor clove_hip_flash_attention(CTensor q, CTensor k, CTensor v, int num_heads, int q_pos,
                                  int k_pos, int flags, float scale) {
    return guarded_tensor([&] {
        return HipBackend::flash_attention(as_node(q), as_node(k), as_node(v), num_heads, q_pos,
                                           k_pos, flags, scale);
    });
}

CTensor clove_hip_rope(CTensor x, size_t pos_offset, size_t head_dim) {
    return guarded_tensor([&] { return HipBackend::rope(as_node(x), pos_offset, head_dim); });
}

int clove_hip_adamw_step(CTensor *weights, CTensor *grads, CTensor *m, CTensor *v, int count,
                         float lr, float beta1, float beta2, float eps, float weight_decay,
                         float loss_scale, float clip, unsigned int step) {
    return guarded([&] {
        if (count < 0) clove::fail(CLOVE_HIP_ERR_INVALID, "adamw: count < 0");
        if (count > 0 && (!weights || !grads || !m || !v))
            clove::fail(CLOVE_HIP_ERR_INVALID, "adamw: a tensor array is NULL");
        std::vector<const Tensor *> w(count), g(count), mm(count), vv(count);
        for (int i = 0; i < count; ++i) {
            w[i] = &deref(weights[i], "weights[i]");
            g[i] = &deref(grads[i], "grads[i]");
            mm[i] = &deref(m[i], "m[i]");
            vv[i] = &deref(v[i], "v[i]");
        }
        HipBackend::adamw_step(w, g, mm, vv,
                               {lr, beta1, beta2, eps, weight_decay, loss_scale, clip, step});
    });
}

CTensor clove_hip_paged_gather_indices(CTensor block_tables, CTensor context_lens, int block_size,
                                       int max_ctx) {
    return guarded_tensor([&] {
        deref(block_tables, "block_tables");
        deref(context_lens, "context_lens");
        return HipBackend::paged_gather_indices(as_node(block_tables), as_node(context_lens),
                                                block_size, max_ctx);
    });
}

// ---- fused chain -----------------------------------------------------------------

int clove_hip_fused_chain(const clove_hip_chain_op *ops, int n_ops, const CTensor *inputs,
                          int n_inputs, CTensor *outputs) {
    int written = 0;
    const int rc = guarded([&] {
        if (!ops || n_ops <= 0) clove::fail(CLOVE_HIP_ERR_INVALID, "no ops");
        if (!inputs || n_inputs <= 0) clove::fail(CLOVE_HIP_ERR_INVALID, "no inputs");
        if (!outputs) clove::fail(CLOVE_HIP_ERR_INVALID, "outputs is NULL");
        std::vector<clove::ChainOp> chain(n_ops);
        for (int i = 0; i < n_ops; ++i) {
            chain[i].opcode = ops[i].opcode;
            chain[i].src0 = ops[i].src0;
            chain[i].src1 = ops[i].src1;
            chain[i].store = ops[i].store != 0 || i + 1 == n_ops;
            chain[i].param = ops[i].param;
        }
        // The structure is checked before anything follows an operand, so
        // the walk below only ever steps to earlier ops and ends at an input.
        clove::validate_chain(chain, (size_t)n_inputs);
        std::vector<const Tensor *> ins(n_inputs);
        for (int k = 0; k < n_inputs; ++k) ins[k] = &deref(inputs[k], "input");
        // Index space: the numel of the last op, which (as in the tracer,
        // lazy.rs:206) is the numel of its first operand, followed back to an
        // input.
        int src = chain.back().src0;
        while (src >= 0) src = chain[src].src0;
        const size_t numel = ins[-src - 1]->numel;
        std::vector<TensorNode> made;
        std::vector<Tensor *> outs;
        for (const auto &op : chain)
            if (op.store) {
                made.push_back(clove::new_tensor(ins[-src - 1]->shape, CLOVE_HIP_F32));
                outs.push_back(made.back().get());
            }
        clove::run_chain(chain, ins, outs, numel);
        for (auto &t : made) outputs[written++] = into_raw(t);
    });
    return rc == CLOVE_HIP_OK ? written : -rc;
}

// ---- graph -------------------------------------------------------------------------

clove_hip_graph *clove_hip_graph_create(void) {
    clove_hip_graph *g = nullptr;
    guarded([&] { g = new clove_hip_graph(); });
    return g;
}

void clove_hip_graph_free(clove_hip_graph *g) { delete g; }

int clove_hip_graph_input(clove_hip_graph *g, const char *shape) {
    int id = -1;
    const int rc = guarded([&] {
        if (!g || !shape) clove::fail(CLOVE_HIP_ERR_INVALID, "graph or shape is NULL");
        id = g->g.add_input(shape);
    });
    return rc == CLOVE_HIP_OK ? id : -rc;
}

int clove_hip_graph_op(clove_hip_graph *g, int opcode, const int *deps, int n_deps, float param) {
    int id = -1;
    const int rc = guarded([&] {
        if (!g) clove::fail(CLOVE_HIP_ERR_INVALID, "graph is NULL");
        if (n_deps < 0 || (n_deps > 0 && !deps)) clove::fail(CLOVE_HIP_ERR_INVALID, "bad operand list");
        id = g->g.add_op(opcode, std::vector<int>(deps, deps + n_deps), param);
    });
    return rc == CLOVE_HIP_OK ? id : -rc;
}

int clove_hip_graph_rope(clove_hip_graph *g, int x, size_t pos_offset, size_t head_dim) {
    int id = -1;
    const int rc = guarded([&] {
        if (!g) clove::fail(CLOVE_HIP_ERR_INVALID, "graph is NULL");
        if (pos_offset >= (1u << 30) || head_dim > 256)
            clove::fail(CLOVE_HIP_ERR_INVALID, "RoPE: pos_offset or head_dim out of range");
        id = g->g.add_rope(x, (int64_t)pos_offset, (int64_t)head_dim);
    });
    return rc == CLOVE_HIP_OK ? id : -rc;
}

clove_hip_model *clove_hip_compile(clove_hip_graph *g, const int *outputs, int n_outputs) {
    clove_hip_model *m = nullptr;
    guarded([&] {
        if (!g || !outputs || n_outputs <= 0) clove::fail(CLOVE_HIP_ERR_INVALID, "bad arguments");
        auto model = std::make_unique<clove_hip_model>();
        model->m = std::make_unique<clove::Model>(g->g, std::vector<int>(outputs, outputs + n_outputs));
        model->description = model->m->describe();
        m = model.release();
    });
    return m;
}

void clove_hip_model_free(clove_hip_model *m) {
    if (!m) return;
    std::lock_guard<std::recursive_mutex> lk(clove::api_mutex());
    delete m;
}

int clove_hip_execute(clove_hip_model *m, const CTensor *inputs, int n_inputs, const int64_t *env,
                      CTensor *outputs) {
    return guarded([&] {
        if (!m || !outputs || (n_inputs > 0 && !inputs)) clove::fail(CLOVE_HIP_ERR_INVALID, "bad arguments");
        std::vector<TensorNode> ins(n_inputs);
        for (int i = 0; i < n_inputs; ++i) {
            deref(inputs[i], "input");
            ins[i] = as_node(inputs[i]);
        }
        std::vector<TensorNode> outs = m->m->execute(ins, env);
        for (size_t i = 0; i < outs.size(); ++i) outputs[i] = into_raw(outs[i]);
    });
}

int clove_hip_model_num_steps(clove_hip_model *m) { return m ? (int)m->m->steps.size() : -1; }

const char *clove_hip_model_describe(clove_hip_model *m) { return m ? m->description.c_str() : ""; }

// ---- timing ----------------------------------------------------------------------------

int clove_hip_event_record(void) {
    int id = -1;
    const int rc = guarded([&] { id = clove::event_record(); });
    return rc == CLOVE_HIP_OK ? id : -rc;
}

int clove_hip_event_elapsed(int a, int b, float *ms) {
    return guarded([&] {
        if (!ms) clove::fail(CLOVE_HIP_ERR_INVALID, "ms is NULL");
        *ms = clove::event_elapsed(a, b);
    });
}

void clove_hip_event_reset(void) {
    guarded([] { clove::event_reset(); });
}

}  // extern "C"
