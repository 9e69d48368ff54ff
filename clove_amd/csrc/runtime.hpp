// runtime.hpp -- context lifecycle, transfers and events (runtime.cpp), and
// the entry points of the fused-chain JIT (jit.cpp), the eager backend
// (ops.cpp) and the lazy planner (graph.cpp).
#pragma once

#include <string>
#include <vector>

#include "common.hpp"

namespace clove {

const std::string &last_error();
void init(int device);
void shutdown();
void synchronize();
void set_stream(void *s);
int32_t *device_error_flag();
// The current device's address of the paged decode's static scratch array
// (k::kPagedScratchFloats floats), taken at init.
float *paged_scratch();

void upload(Tensor &t, const void *src, size_t offset, size_t count);
void download(const Tensor &t, void *dst, size_t offset, size_t count);

int event_record();
float event_elapsed(int a, int b);
void event_reset();

void fill_normal(Tensor &t, uint64_t seed, float mean, float stddev);
void fill_uniform(Tensor &t, uint64_t seed, float lo, float hi);

// ---- fused elementwise chains (jit.cpp) ----------------------------------

// One op of a chain; operands >= 0 name earlier ops, < 0 name input -(x+1).
struct ChainOp {
    int opcode;
    int src0 = 0, src1 = 0;
    bool store = false;
    float param = 0.f;
};

// Number of operands an elementwise opcode reads (1 or 2); 0 if the opcode
// is not elementwise.
int ew_arity(int opcode);

// Checks a chain's structure: 1..CL_MAX_OPS elementwise ops, 1..CL_MAX_IN
// inputs, every operand an earlier op or an existing input, at most
// CL_MAX_OUT stored values (the last op always is).  Returns the number of
// stored values; fails with CLOVE_HIP_ERR_INVALID otherwise.
int validate_chain(const std::vector<ChainOp> &ops, size_t n_inputs);

// Evaluates `ops` over the index space [0, numel) and writes the stored ops
// into `outs` (one pre-allocated f32 tensor of at least numel elements per
// stored op, in op order).
void run_chain(const std::vector<ChainOp> &ops, const std::vector<const Tensor *> &inputs,
               const std::vector<Tensor *> &outs, size_t numel);
void jit_shutdown();
// Drops the cached RoPE tables (attention.cpp); part of shutdown.
void rope_cache_clear();
// Diagnostics for tests: number of chains compiled so far.
int jit_compiled_count();
// Chains compiled with hipRTC and chains loaded from the on-disk cache by
// this process so far.
void jit_stats(int *compiled, int *disk_loads);

// ---- eager backend (ops.cpp): mirrors trait Backend (backend.rs:171-257) --

struct HipBackend {
    static TensorNode new_cpu(const float *data, const std::vector<size_t> &shape);
    static TensorNode binary(int opcode, const TensorNode &a, const TensorNode &b);
    static TensorNode unary(int opcode, const TensorNode &a, float param = 0.f);
    static TensorNode add(const TensorNode &a, const TensorNode &b);
    static TensorNode sub(const TensorNode &a, const TensorNode &b);
    static TensorNode mul(const TensorNode &a, const TensorNode &b);
    static TensorNode mul_scalar(const TensorNode &a, float s);
    static TensorNode transpose(const TensorNode &a);
    static TensorNode flatten(const TensorNode &a);
    static TensorNode concat_seq(const TensorNode &a, const TensorNode &b);
    static TensorNode relu(const TensorNode &a);
    static TensorNode gelu(const TensorNode &a);
    static TensorNode sigmoid(const TensorNode &a);
    static TensorNode tanh(const TensorNode &a);
    static TensorNode sin(const TensorNode &a);
    static TensorNode cos(const TensorNode &a);
    static TensorNode softmax(const TensorNode &a);
    static TensorNode layer_norm(const TensorNode &a, const TensorNode &gamma,
                                 const TensorNode &beta);
    static TensorNode matmul(const TensorNode &a, const TensorNode &b);
    static TensorNode paged_attention(const TensorNode &q, const TensorNode &k,
                                      const TensorNode &v, const TensorNode &kv_cache,
                                      const TensorNode &block_tables,
                                      const TensorNode &context_lens, float scale);
    // Paged decode on caller-owned device memory with the partition
    // workspace in the static scratch array: no device allocation.
    struct PagedRaw {
        const float *q, *k_new, *v_new, *kv_cache;
        int64_t num_blocks;
        int block_size, num_heads, head_dim;
        const int32_t *block_tables;
        int max_blocks;
        const int32_t *context_lens;
        int num_seqs;
        float scale;
        float *out;
    };
    static void paged_attention_noalloc(const PagedRaw &r);
    static void paged_kv_append(const Tensor &kv_cache, const Tensor &k, const Tensor &v,
                                const Tensor &block_tables, const Tensor &context_lens);
    static TensorNode paged_gather_indices(const TensorNode &block_tables,
                                           const TensorNode &context_lens, int block_size,
                                           int max_ctx);

    // Backward passes and losses (grad.cpp; the autograd closures of
    // backend.rs).
    static TensorNode relu_backward(const TensorNode &x, const TensorNode &grad_out);
    static TensorNode gelu_backward(const TensorNode &x, const TensorNode &grad_out);
    static TensorNode softmax_backward(const TensorNode &y, const TensorNode &grad_out);
    static void matmul_backward(const TensorNode &a, const TensorNode &b, const TensorNode &grad_out,
                                TensorNode *grad_a, TensorNode *grad_b);
    static TensorNode broadcast_grad(const TensorNode &grad_out, size_t b_numel, bool negate);
    static TensorNode cross_entropy(const TensorNode &logits, const TensorNode &targets);
    static TensorNode cross_entropy_backward(const TensorNode &logits, const TensorNode &targets,
                                             const TensorNode &grad_loss);
    static TensorNode mse(const TensorNode &pred, const TensorNode &target);
    static TensorNode mse_backward(const TensorNode &pred, const TensorNode &target,
                                   const TensorNode &grad_loss);
    // Attention prefill and RoPE (attention.cpp).
    static TensorNode flash_attention(const TensorNode &q, const TensorNode &k,
                                      const TensorNode &v, int num_heads, int q_pos, int k_pos,
                                      int flags, float scale);
    static TensorNode rope(const TensorNode &x, size_t pos_offset, size_t head_dim);
    static void rope_into(const Tensor &x, size_t pos_offset, size_t head_dim, Tensor &out);
    // RoPE at (q_pos, k_pos); key t is hidden from query s when causal and
    // t + mask_k > s + mask_q.
    static void flash_attention_into(const Tensor &q, const Tensor &k, const Tensor &v,
                                     int num_heads, int q_pos, int k_pos, int mask_q, int mask_k,
                                     int flags, float scale, Tensor &out);
    // optim.rs:375-395: one AdamW step in place on every (w, g, m, v).
    struct AdamWParams {
        float lr, beta1, beta2, eps, weight_decay, loss_scale, clip;
        uint32_t step;
    };
    static void adamw_step(const std::vector<const Tensor *> &w,
                           const std::vector<const Tensor *> &g,
                           const std::vector<const Tensor *> &m,
                           const std::vector<const Tensor *> &v, const AdamWParams &p);

    // Launch-only forms writing into caller-provided outputs (used by the
    // planner, whose buffers are pre-assigned).
    static void softmax_into(const Tensor &a, Tensor &out);
    static void layer_norm_into(const Tensor &a, const Tensor &gamma, const Tensor &beta,
                                Tensor &out);
    // Optional fused epilogue: out = act(a.b + bias[i % numel(bias)]) with
    // act 0 none, 1 ReLU, 2 GELU (CLOVE_OP_* elementwise semantics).
    static void matmul_into(const Tensor &a, const Tensor &b, Tensor &out,
                            const Tensor *bias = nullptr, int act = 0);
    // One member of a horizontal MatMul group: out = act(a.b + bias).
    struct GemmMember {
        const Tensor *a, *b;
        Tensor *out;
        const Tensor *bias;
        int act;
    };
    static void matmul_group_into(const std::vector<GemmMember> &members);
    static void paged_attention_into(const Tensor &q, const Tensor *k, const Tensor *v,
                                     const Tensor &kv_cache, const Tensor &block_tables,
                                     const Tensor &context_lens, float scale, Tensor &out);
};

}  // namespace clove
