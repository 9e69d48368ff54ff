// launch.hpp -- host-side launchers of the ahead-of-time gfx950 kernels.
// Each launcher validates nothing: shape checks happen in ops.cpp before a
// launcher is called, so every launcher assumes its arguments are in range.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace clove {
namespace k {

// fill.hip -- seeded synthetic data (counter-based splitmix64 stream).
void fill_normal(float *p, size_t n, uint64_t seed, float mean, float stddev, hipStream_t s);
void fill_uniform(float *p, size_t n, uint64_t seed, float lo, float hi, hipStream_t s);

// rowwise.hip -- one wavefront per row, the row held in registers.
void softmax_rows(const float *x, float *y, size_t rows, size_t cols, hipStream_t s);
void layer_norm_rows(const float *x, const float *gamma, const float *beta, float *y,
                     size_t rows, size_t cols, float eps, hipStream_t s);

// Backward rows (rowwise.hip): softmax backward and cross entropy.  The
// cross-entropy kernels read f32 class indices for the first `used` rows; a
// class >= cols sets *err_flag.  cross_entropy_rows writes one value per row
// ((l[t] - max) - ln(sum exp)), which ordered_sum turns into the loss.
void softmax_backward_rows(const float *y, const float *dy, float *dx, size_t rows, size_t cols,
                           hipStream_t s);
void cross_entropy_rows(const float *logits, const float *targets, size_t used, size_t rows,
                        size_t cols, float *row_values, int *err_flag, hipStream_t s);
void cross_entropy_backward_rows(const float *logits, const float *targets, size_t used,
                                 size_t rows, size_t cols, const float *grad_loss, float *grad,
                                 int *err_flag, hipStream_t s);

// reduce.hip -- deterministic reductions and the transpose.
// gb[j] = (negate ? -1 : 1) * sum_{i % nb == j} g[i]; part holds
// broadcast_grad_workspace(n, nb) floats.
size_t broadcast_grad_workspace(size_t n, size_t nb);
void broadcast_grad(const float *g, size_t n, size_t nb, bool negate, float *part, float *gb,
                    hipStream_t s);
// out[0] = sum((p - t)^2) / n; part holds sq_diff_workspace(n) floats.
size_t sq_diff_workspace(size_t n);
void mse_loss(const float *p, const float *t, size_t n, float *part, float *out, hipStream_t s);
void mse_backward(const float *p, const float *t, size_t n, const float *grad_loss, float *grad,
                  hipStream_t s);
// out[0] = (sign * sum of x[0..n)) / div, summed in a fixed order.
void ordered_sum(const float *x, size_t n, float sign, float div, float *out, hipStream_t s);
// out[C][R] = in[R][C].
void transpose(const float *in, float *out, size_t R, size_t C, hipStream_t s);

// flash_attention.hip -- attention prefill and RoPE.  q [B, S, H*D], k, v
// [B, Sk, H*D], out [B, S, H*D]; D in [1, kAttnMaxHeadDim].  D 64 and 128
// run fixed-shape kernels, every other D the general one; all four tensors
// 16-byte aligned when D % 4 == 0, else 4-byte aligned with a null
// q_rope_tab (the caller rotates q first).
constexpr int kAttnMaxHeadDim = 256;
bool attention_supported(int head_dim);
// q_rope_tab: a (cos, sin) table (rope_table layout) whose rows cover
// positions q_pos .. q_pos + S - 1 from tab_pos0, to rotate q inside the
// kernel, or null (k must then already be rotated by the caller when RoPE
// applies).
void attention_prefill(const float *q, const float *k, const float *v, float *out, int B, int S,
                       int Sk, int H, int D, int q_pos, int k_pos, bool causal, float scale,
                       const float *q_rope_tab, int tab_pos0, hipStream_t s);
// freq.div[j] = 10000^(2j / D) (powf on the host, as backend.rs:2818 forms it).
struct AttnFreq {
    float div[128];
};
// tab (npos * head_dim/2 float pairs): (cos, sin) of (pos0 + p) / div[j].
void rope_table(float *tab, int pos0, int npos, int head_dim, const AttnFreq &freq,
                hipStream_t s);
// x [rows, hidden], rows = batch * seq: pairs of each whole head_dim-wide head
// rotated at position (row % seq) + pos_offset (the table row
// pos - tab_pos0); dims past the last whole head are written as 0.
void rope_apply(const float *x, float *out, size_t rows, int seq, int hidden, int head_dim,
                int pos_offset, const float *tab, int tab_pos0, hipStream_t s);

// optim.hip -- the fused AdamW update, in place on w, m, v, for `count`
// parameter tensors (kAdamWMaxTensors per launch).  bias1 / bias2 are
// 1 - beta1^t and 1 - beta2^t.
constexpr int kAdamWMaxTensors = 16;
struct AdamWHyper {
    float lr, beta1, beta2, eps, weight_decay, loss_scale, clip, bias1, bias2;
};
void adamw_step(float *const *w, const float *const *g, float *const *m, float *const *v,
                const uint64_t *n, int count, const AdamWHyper &h, int num_cus, hipStream_t s);

// gemm_f32.hip -- C[M,N] = A[M,K] . B[K,N], row-major f32, MFMA f32 accumulate.
struct GemmPlan {
    int M, N, K;
    int cfg;           // tile configuration
    int tiles, tiles_n;
    int splits;        // K splits across workgroups (1: no workspace)
    int k_per_split;   // multiple of the configuration's K slab
    size_t ws_floats;  // split-K workspace
    bool vec, interior;
    // Skinny path (M <= 64): one workgroup of `waves` waves per 32*nb
    // columns and K split; each wave streams its own k_per_wave range of B.
    bool skinny;
    int mb;            // 32-row blocks per wave (1 or 2)
    int nb;            // 32-column blocks per wave (1, 2 or 4)
    int waves;         // waves per workgroup (K split inside the workgroup)
    int k_per_wave;    // a whole number of pipeline chunks
    // Small path: one workgroup of `waves` waves per 16 x 16 tile of C, K
    // split inside the workgroup (k_per_split k per wave); no workspace.
    bool small;
    // Strip path (M <= 32): one workgroup per 16-row half of a 32-column
    // strip over the whole K (k_per_wave k per wave, `waves` waves); one
    // launch, no workspace.  tiles_n = strips, tiles = halves * strips.
    bool strip;
};
// Optional epilogue fused into the GEMM store: bias add with Clove's
// broadcast rule (bias read at flat index % bias_n) and an activation.
enum { GEMM_BIAS_NONE = 0, GEMM_BIAS_COL = 1, GEMM_BIAS_SCALAR = 2, GEMM_BIAS_MOD = 3 };
// GEMM_ACT_SOFTMAX is a row softmax over the last dimension after the bias;
// only the small path with N <= 16 (one tile column holds whole rows) applies
// it in the kernel; matmul_into runs a separate row softmax otherwise.
enum { GEMM_ACT_NONE = 0, GEMM_ACT_RELU = 1, GEMM_ACT_GELU = 2, GEMM_ACT_SOFTMAX = 3 };
struct GemmEpilogue {
    const float *bias = nullptr;
    uint64_t bias_n = 0;
    int bias_mode = GEMM_BIAS_NONE;
    int act = GEMM_ACT_NONE;
};
// Independent small-path products in one launch (the planner's horizontal
// MatMul groups): at most kGemmGroupMax; every plan must be small and a
// softmax epilogue needs N <= 16.
constexpr int kGemmGroupMax = 8;
void gemm_f32_grouped(const GemmPlan *plans, const float *const *A, const float *const *B,
                      float *const *C, const GemmEpilogue *epi, int count, hipStream_t s);
// Picks the tile configuration and K split for a shape.  a_aligned / b_aligned:
// A / B is 16-byte aligned (the small path needs A aligned, the strip and
// skinny paths both, as they read them in 8- and 16-byte vectors).
// force_cfg >= 0 overrides the
// configuration and turns the skinny path off; force_skinny takes the skinny
// path wherever it is legal, with force_skinny_nb (1, 2, 4) /
// force_skinny_splits > 0 overriding its plan; force_strip takes the strip
// path wherever it is legal (M <= 32, even N, K % 4 == 0, K <= 16384; tuning
// and tests).  Every plan computes the same product.
GemmPlan gemm_plan(int M, int N, int K, int num_cus, int force_cfg, bool a_aligned = true,
                   bool force_skinny = false, int force_skinny_nb = 0,
                   int force_skinny_splits = 0, bool force_strip = false,
                   bool b_aligned = true);
void gemm_f32(const GemmPlan &p, const float *A, const float *B, float *C, float *ws,
              const GemmEpilogue &epi, hipStream_t s);
// C = A^T . B (ta: A holds the [K, M] matrix) or C = A . B^T (tb: B holds the
// [N, K] matrix), read transposed inside the tiled kernel's slab loads: the
// same bits as transposing first.  ws: p.ws_floats floats when p splits K.
// Launches nothing and returns false unless exactly one of ta, tb is set and
// p is a 128x128 or 128x256 tiled plan, or a 64x128 one the DMA kernel takes,
// with 16-byte aligned operands whose transposed rows hold whole 16-byte
// pieces where its tiles are ragged; the caller then transposes explicitly.
bool gemm_f32_transposed(const GemmPlan &p, const float *A, const float *B, float *C, float *ws,
                         bool ta, bool tb, hipStream_t s);

// Bits of the device error word (runtime.cpp) that the next synchronising
// call reports: kernels OR them in when they meet a bad index.
enum : int32_t {
    kErrPagedRange = 1,  // a block-table entry outside the pool / a context past the table
    kErrClassRange = 2,  // a cross-entropy target >= the number of classes
    kErrIndexValue = 4,  // an f32 index tensor held a value that is not an integer in [0, 2^24)
};

// paged_attention.hip
struct PagedArgs {
    const float *q;        // [B, H, D]
    const float *k_new;    // [B, H, D] or nullptr
    const float *v_new;    // [B, H, D] or nullptr
    const float *k_cache;  // [num_blocks, block_size, H, D]
    const float *v_cache;  // [num_blocks, block_size, H, D]
    const int32_t *block_tables;  // [B, max_blocks]
    const int32_t *context_lens;  // [B]
    float *out;            // [B, H, D]
    float *partials;       // workspace: [B, H, max_parts, D + 2]
    int32_t *err_flag;     // set to 1 when a table entry used lies outside the pool
    int64_t num_blocks;    // blocks in the pool (bounds for table entries)
    int num_seqs, num_heads, head_dim, block_size, max_blocks, max_parts;
    int part_tokens;       // tokens per partition (multiple of block_size)
    int gen_shift;         // general kernel: line-aligned pieces (set by paged_attention)
    float scale;
};
// The allocation-free decode's partition workspace: a static device array
// of this many floats (16 MiB) in paged_attention.hip.  paged_scratch_address
// returns its address on the current device (call it with each device
// current once; the address differs per device).
constexpr size_t kPagedScratchFloats = size_t(4) << 20;
hipError_t paged_scratch_address(float **ptr);
// Workspace floats needed for a given shape (0 when one partition suffices).
size_t paged_workspace_floats(int num_seqs, int num_heads, int head_dim, int max_ctx,
                              int part_tokens);
int paged_part_tokens(int num_seqs, int num_heads, int capacity, int block_size, int num_cus);
// Head dims 64/128/256 with block sizes 8/16/32 run a fixed-shape kernel;
// every other head_dim in [1, kPagedMaxHeadDim] and block size >= 1 runs
// the general one.
constexpr int kPagedMaxHeadDim = 1024;
bool paged_supported(int head_dim, int block_size);
void paged_attention(const PagedArgs &a, hipStream_t s);
// row_floats = H * D (a multiple of 4); k_new/v_new are [B, row_floats].
void paged_append(float *k_cache, float *v_cache, const float *k_new, const float *v_new,
                  const int32_t *block_tables, const int32_t *context_lens, int num_seqs,
                  int max_blocks, int block_size, int64_t num_blocks, int row_floats,
                  int32_t *err_flag, hipStream_t s);
// Slots bt[b][t/bs]*bs + t%bs, -1 past ctx_b; a negative entry, or one
// whose slots do not fit in int32, gives -1 and sets kErrPagedRange.
void paged_slots(const int32_t *block_tables, const int32_t *context_lens, int32_t *slots,
                 int num_seqs, int max_blocks, int block_size, int max_ctx, int32_t *err_flag,
                 hipStream_t s);
// Block tables / context lengths that arrive as f32 (Clove builds every
// tensor from a Vec<f32>, backend.rs:176), converted in one launch.  A value
// is taken when it is an integer in [0, 2^24), where f32 holds every integer
// exactly; otherwise it becomes -1.  A bad context length always sets
// kErrIndexValue; a bad table entry only when its sequence's context reaches
// it (entry j of sequence b is used when j * block_size < ctx_b), so padding
// past a sequence's blocks is never an error, as it is never read.
//   bt_f  f32 [B, max_blocks] or null (the table is int32 already)
//   cl_f  f32 [B] or null, in which case cl_i (int32 [B]) gives the lengths
void paged_index_from_f32(const float *bt_f, int32_t *bt_out, const float *cl_f,
                          const int32_t *cl_i, int32_t *cl_out, int num_seqs, int max_blocks,
                          int block_size, int32_t *err_flag, hipStream_t s);

}  // namespace k
}  // namespace clove
