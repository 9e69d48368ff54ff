// paged_attention.hip -- PagedAttention decode over block tables.
//
// Reference: the op contract of Backend::paged_attention (backend.rs:249-256,
// ffi.rs:247-266), the cache / table layout documented at nn.rs:534-535 and
// the block-table gather of the lazy WGSL (lazy.rs:5262-5270).  That WGSL is
// a placeholder (out = q * k * scale, no softmax, no V), so the arithmetic
// here is the textbook decode: per (sequence b, head h)
//   out = sum_t softmax_t(scale * q . K_t) V_t,  t = 0 .. ctx_b - 1,
// where token t lives in physical slot bt[b][t / bs] * bs + t % bs of the
// pool and, when a new token's k/v are passed, token ctx_b - 1 is read from
// them.
//
// Work split (flash-decoding): the context of each (b, h) is cut into
// partitions of `part_tokens` tokens (a whole number of KV blocks).  One
// workgroup of four waves handles one (partition, h, b); the waves take the
// partition's KV blocks round-robin.  Within a wave a token's head vector
// (D floats) is spread over D/4 lanes as 16-byte loads, so one wave load
// instruction reads 64/(D/4) whole token rows (two 512-byte rows for
// D = 128) and every byte fetched is used.  q.k is reduced across those
// lanes with butterflies; the online softmax keeps (max, sum, acc) per wave,
// the waves are merged through LDS, and a partition's (max, sum, acc) goes
// to a workspace that a second kernel merges with the log-sum-exp rule.
// A sequence that fits one partition is written directly.
//
// Safety: context lengths are clamped to the table's capacity and table
// entries outside [0, num_blocks) are skipped; both set a device error flag
// that the host reports at its next synchronisation point.  No load is ever
// issued outside the pool.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "launch.hpp"
#include "wave.h"

namespace clove {
namespace k {

namespace {

// Physical slot of logical token t of a sequence whose table row is `bt`.
__device__ __forceinline__ int64_t paged_slot(const int32_t *bt, int t, int bs) {
    return (int64_t)bt[t / bs] * bs + t % bs;
}

__device__ __forceinline__ int clamp_ctx(const PagedArgs &a, int b, bool report) {
    int ctx = a.context_lens[b];
    const int cap = a.max_blocks * a.block_size;
    if (ctx < 0 || ctx > cap) {
        if (report) atomicOr(a.err_flag, 1);
        ctx = ctx < 0 ? 0 : cap;
    }
    return ctx;
}

template <int D, int BS>
__global__ void __launch_bounds__(256) paged_partition_kernel(PagedArgs a) {
    constexpr int LPT = D / 4;      // lanes per token row
    constexpr int TPL = 64 / LPT;   // token rows per wave load
    constexpr int STEPS = BS / TPL; // wave loads per KV block
    static_assert(BS % TPL == 0, "block size must be a multiple of the rows per load");
    __shared__ float s_o[4][D];
    __shared__ float s_m[4], s_l[4];

    const int part = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ctx = clamp_ctx(a, b, part == 0 && h == 0 && threadIdx.x == 0);
    const int t_begin = part * a.part_tokens;
    if (t_begin >= ctx) return;
    const int t_end = min(t_begin + a.part_tokens, ctx);
    const int H = a.num_heads;
    const int sub = lane / LPT;     // which token row of a load group
    const int dl = lane % LPT;      // 16-byte column within the row

    const size_t head_off = ((size_t)b * H + h) * D;
    const cl_f4 q = *reinterpret_cast<const cl_f4 *>(a.q + head_off + 4 * dl);
    const int32_t *bt = a.block_tables + (size_t)b * a.max_blocks;
    const bool has_new = a.k_new != nullptr;
    const size_t row_stride = (size_t)H * D;  // floats between consecutive slots

    float m = -INFINITY, l = 0.0f;
    cl_f4 o = {0.f, 0.f, 0.f, 0.f};

    const int lb_first = t_begin / BS, lb_last = (t_end - 1) / BS;
    for (int lb = lb_first + wave; lb <= lb_last; lb += 4) {
        const int64_t blk = bt[lb];
        if (blk < 0 || blk >= a.num_blocks) {
            if (lane == 0) atomicOr(a.err_flag, 1);
            continue;
        }
        const size_t blk_off = (size_t)blk * BS * row_stride + (size_t)h * D + 4 * dl;
        const float *kbase = a.k_cache + blk_off;
        const float *vbase = a.v_cache + blk_off;
        // All K rows of the block are loaded before any is used.
        cl_f4 kv[STEPS];
        bool in[STEPS];
#pragma unroll
        for (int st = 0; st < STEPS; ++st) {
            const int r = st * TPL + sub;
            const int t = lb * BS + r;
            in[st] = t >= t_begin && t < t_end;
            kv[st] = (cl_f4){0.f, 0.f, 0.f, 0.f};
            if (in[st]) {
                const float *kp = (has_new && t == ctx - 1) ? a.k_new + head_off + 4 * dl
                                                            : kbase + (size_t)r * row_stride;
                kv[st] = *reinterpret_cast<const cl_f4 *>(kp);
            }
        }
        float sc[STEPS];
        float bm = -INFINITY;
#pragma unroll
        for (int st = 0; st < STEPS; ++st) {
            float d = (q.x * kv[st].x + q.y * kv[st].y) + (q.z * kv[st].z + q.w * kv[st].w);
#pragma unroll
            for (int off = LPT / 2; off > 0; off >>= 1) d += __shfl_xor(d, off, 64);
            sc[st] = in[st] ? d * a.scale : -INFINITY;
            bm = fmaxf(bm, sc[st]);
        }
#pragma unroll
        for (int off = LPT; off < 64; off <<= 1) bm = fmaxf(bm, __shfl_xor(bm, off, 64));
        const float m_new = fmaxf(m, bm);
        const float alpha = (m == -INFINITY) ? 0.0f : expf(m - m_new);
        l *= alpha;
        o *= alpha;
        cl_f4 vv[STEPS];
#pragma unroll
        for (int st = 0; st < STEPS; ++st) {
            const int r = st * TPL + sub;
            const int t = lb * BS + r;
            vv[st] = (cl_f4){0.f, 0.f, 0.f, 0.f};
            if (in[st]) {
                const float *vp = (has_new && t == ctx - 1) ? a.v_new + head_off + 4 * dl
                                                            : vbase + (size_t)r * row_stride;
                vv[st] = *reinterpret_cast<const cl_f4 *>(vp);
            }
        }
#pragma unroll
        for (int st = 0; st < STEPS; ++st) {
            if (in[st]) {
                const float p = expf(sc[st] - m_new);
                l += p;
                o += p * vv[st];
            }
        }
        m = m_new;
    }

    // Merge the token-row groups of the wave (same running max in all lanes).
#pragma unroll
    for (int off = LPT; off < 64; off <<= 1) {
        l += __shfl_xor(l, off, 64);
        o.x += __shfl_xor(o.x, off, 64);
        o.y += __shfl_xor(o.y, off, 64);
        o.z += __shfl_xor(o.z, off, 64);
        o.w += __shfl_xor(o.w, off, 64);
    }
    if (sub == 0) *reinterpret_cast<cl_f4 *>(&s_o[wave][4 * dl]) = o;
    if (lane == 0) {
        s_m[wave] = m;
        s_l[wave] = l;
    }
    __syncthreads();

    // Merge the four waves: thread d < D owns output element d.
    const int d = threadIdx.x;
    if (d < D) {
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; ++w) M = fmaxf(M, s_m[w]);
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            if (s_m[w] == -INFINITY) continue;
            const float e = expf(s_m[w] - M);
            L += s_l[w] * e;
            O += s_o[w][d] * e;
        }
        if (ctx <= a.part_tokens) {
            a.out[head_off + d] = O / L;
        } else {
            float *p = a.partials + (((size_t)b * H + h) * a.max_parts + part) * (D + 2);
            p[d] = O;
            if (d == 0) {
                p[D] = M;
                p[D + 1] = L;
            }
        }
    }
}

// Merges the partitions of each (b, h): out = sum_p O_p e^(M_p - M) /
// sum_p L_p e^(M_p - M).  Also writes zeros for empty contexts.
__global__ void __launch_bounds__(256) paged_merge_kernel(PagedArgs a) {
    const int h = blockIdx.x, b = blockIdx.y;
    const int D = a.head_dim;
    const int d = threadIdx.x;
    if (d >= D) return;
    const int ctx = clamp_ctx(a, b, false);
    const size_t head_off = ((size_t)b * a.num_heads + h) * D;
    if (ctx <= 0) {
        a.out[head_off + d] = 0.0f;
        return;
    }
    const int parts = (ctx + a.part_tokens - 1) / a.part_tokens;
    if (parts <= 1) return;
    const float *p = a.partials + ((size_t)b * a.num_heads + h) * a.max_parts * (D + 2);
    float M = -INFINITY;
    for (int i = 0; i < parts; ++i) M = fmaxf(M, p[i * (D + 2) + D]);
    float L = 0.0f, O = 0.0f;
    for (int i = 0; i < parts; ++i) {
        const float mi = p[i * (D + 2) + D];
        if (mi == -INFINITY) continue;
        const float e = expf(mi - M);
        L += p[i * (D + 2) + D + 1] * e;
        O += p[i * (D + 2) + d] * e;
    }
    a.out[head_off + d] = O / L;
}

__global__ void __launch_bounds__(256) paged_slots_kernel(const int32_t *__restrict__ bt,
                                                          const int32_t *__restrict__ cl,
                                                          int32_t *__restrict__ slots,
                                                          int num_seqs, int max_blocks, int bs,
                                                          int max_ctx) {
    const int64_t total = (int64_t)num_seqs * max_ctx;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * 256) {
        const int b = (int)(i / max_ctx), t = (int)(i % max_ctx);
        const int ctx = cl[b];
        slots[i] = (t < ctx && t < max_blocks * bs)
                       ? (int32_t)paged_slot(bt + (size_t)b * max_blocks, t, bs)
                       : -1;
    }
}

}  // namespace

bool paged_supported(int head_dim, int block_size) {
    return (head_dim == 64 || head_dim == 128 || head_dim == 256) &&
           (block_size == 8 || block_size == 16 || block_size == 32);
}

int paged_part_tokens(int head_dim, int block_size) {
    (void)head_dim;
    int blocks = 512 / block_size;
    if (blocks < 1) blocks = 1;
    return blocks * block_size;
}

size_t paged_workspace_floats(int num_seqs, int num_heads, int head_dim, int max_ctx,
                              int part_tokens) {
    const int parts = (max_ctx + part_tokens - 1) / part_tokens;
    if (parts <= 1) return 0;
    return (size_t)num_seqs * num_heads * parts * (head_dim + 2);
}

void paged_attention(const PagedArgs &a, hipStream_t s) {
    if (a.num_seqs <= 0 || a.num_heads <= 0) return;
    const dim3 grid((unsigned)a.max_parts, (unsigned)a.num_heads, (unsigned)a.num_seqs);
#define CLOVE_PAGED_CASE(D, BS)                                              \
    if (a.head_dim == D && a.block_size == BS) {                             \
        paged_partition_kernel<D, BS><<<grid, 256, 0, s>>>(a);               \
    } else
    CLOVE_PAGED_CASE(64, 8) CLOVE_PAGED_CASE(64, 16) CLOVE_PAGED_CASE(64, 32)
    CLOVE_PAGED_CASE(128, 8) CLOVE_PAGED_CASE(128, 16) CLOVE_PAGED_CASE(128, 32)
    CLOVE_PAGED_CASE(256, 8) CLOVE_PAGED_CASE(256, 16) CLOVE_PAGED_CASE(256, 32)
    { return; }
#undef CLOVE_PAGED_CASE
    paged_merge_kernel<<<dim3((unsigned)a.num_heads, (unsigned)a.num_seqs), 256, 0, s>>>(a);
}

void paged_slots(const int32_t *block_tables, const int32_t *context_lens, int32_t *slots,
                 int num_seqs, int max_blocks, int block_size, int max_ctx, hipStream_t s) {
    const int64_t total = (int64_t)num_seqs * max_ctx;
    if (total <= 0) return;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    paged_slots_kernel<<<(unsigned)blocks, 256, 0, s>>>(block_tables, context_lens, slots,
                                                        num_seqs, max_blocks, block_size, max_ctx);
}

}  // namespace k
}  // namespace clove
