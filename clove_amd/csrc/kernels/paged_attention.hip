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
// Work split (flash-decoding).  The context of each (b, h) is cut into
// partitions of `part_tokens` tokens (a whole number of KV blocks).  One
// workgroup of four waves handles one (partition, h, b); its waves take the
// partition's KV blocks round-robin.
//
// Lane layout.  A token's head row (D floats, contiguous) belongs to one
// 16-lane DPP row of the wave: lane c of the row holds the 16-byte pieces
// at floats 4c, 64+4c, ... (D/64 pieces).  One wave load therefore reads
// four whole token rows in 256-byte contiguous runs, every byte fetched is
// used, and q.k is reduced inside the DPP row with four full-rate
// v_add_f32_dpp (quad_perm 1032, quad_perm 2301, row_ror 4, row_ror 8) --
// no LDS traffic.  A KV block (16 tokens) is 4 such loads for K and 4 for
// V per piece; all of them are issued before any arithmetic so a wave keeps
// 16 KiB in flight.  Only the block that holds token ctx-1 can be partial
// or carry the new token; it alone takes the per-token checked path.
//
// Softmax.  Each wave keeps a running (max, sum, acc) (online softmax); the
// four waves are merged through LDS; a partition's (max, sum, acc) goes to a
// workspace, and the LAST workgroup of the (b, h) to finish (an atomic
// ticket per (b, h)) merges the partitions with the log-sum-exp rule and
// writes the output.  The ticket counters reset themselves, so they are zero
// at the start of every launch.  exp is the hardware 2^x of x*log2(e)
// (relative error ~1e-6, far below the 2e-3 parity bound).
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

__device__ __forceinline__ float fast_exp(float x) {
    return __builtin_amdgcn_exp2f(x * 1.44269504088896341f);
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over the 16 lanes of a DPP row; every lane of the row gets the sum.
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp<0x124>(v);  // row_ror 4
    v += dpp<0x128>(v);  // row_ror 8
    return v;
}

__device__ __forceinline__ float dot4(cl_f4 a, cl_f4 b) {
    return (a.x * b.x + a.y * b.y) + (a.z * b.z + a.w * b.w);
}

struct WaveState {
    float m, l;
};

// Folds one KV block into the wave's running softmax state.  `kb`/`vb`
// point at this lane's first piece of the block's row `row`; rows advance
// by 4 per step.  CHECKED handles a partial block and the new-token row.
template <int D, int BS, bool CHECKED>
__device__ __forceinline__ void fold_block(const PagedArgs &a, const float *kb, const float *vb,
                                           size_t row_stride, int t0, int t_end, int ctx,
                                           int row, size_t new_off, const cl_f4 (&q)[D / 64],
                                           WaveState &st, cl_f4 (&o)[D / 64]) {
    constexpr int NV = D / 64;
    constexpr int STEPS = BS / 4;
    cl_f4 kk[STEPS][NV], vv[STEPS][NV];
    bool in[STEPS];
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
        const int t = t0 + 4 * s + row;
        in[s] = !CHECKED || t < t_end;
        const bool fresh = CHECKED && a.k_new != nullptr && t == ctx - 1;
        const float *kp = fresh ? a.k_new + new_off : kb + (size_t)(4 * s) * row_stride;
        const float *vp = fresh ? a.v_new + new_off : vb + (size_t)(4 * s) * row_stride;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            if (in[s]) {
                kk[s][j] = *reinterpret_cast<const cl_f4 *>(kp + 64 * j);
                vv[s][j] = *reinterpret_cast<const cl_f4 *>(vp + 64 * j);
            } else {
                kk[s][j] = (cl_f4){0.f, 0.f, 0.f, 0.f};
                vv[s][j] = (cl_f4){0.f, 0.f, 0.f, 0.f};
            }
        }
    }
    float sc[STEPS];
    float bm = -INFINITY;
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
        float d = dot4(q[0], kk[s][0]);
#pragma unroll
        for (int j = 1; j < NV; ++j) d += dot4(q[j], kk[s][j]);
        d = row16_sum(d);
        sc[s] = in[s] ? d * a.scale : -INFINITY;
        bm = fmaxf(bm, sc[s]);
    }
    bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
    bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
    const float m_new = fmaxf(st.m, bm);
    const float alpha = (st.m == -INFINITY) ? 0.0f : fast_exp(st.m - m_new);
    st.l *= alpha;
#pragma unroll
    for (int j = 0; j < NV; ++j) o[j] *= alpha;
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
        const float p = in[s] ? fast_exp(sc[s] - m_new) : 0.0f;
        st.l += p;
#pragma unroll
        for (int j = 0; j < NV; ++j) o[j] += p * vv[s][j];
    }
    st.m = m_new;
}

template <int D, int BS>
__global__ void __launch_bounds__(256) paged_partition_kernel(PagedArgs a) {
    constexpr int NV = D / 64;
    static_assert(BS % 4 == 0 && D % 64 == 0, "4 rows per wave load, 64 floats per piece row");
    __shared__ float s_o[4][D];
    __shared__ float s_m[4], s_l[4];
    __shared__ int s_last;

    const int part = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row = lane >> 4, c16 = lane & 15;
    const int H = a.num_heads;
    const size_t head_off = ((size_t)b * H + h) * D;
    const int ctx = clamp_ctx(a, b, part == 0 && h == 0 && threadIdx.x == 0);
    const int t_begin = part * a.part_tokens;
    if (t_begin >= ctx) {
        if (ctx == 0 && part == 0 && (int)threadIdx.x < D) a.out[head_off + threadIdx.x] = 0.0f;
        return;
    }
    const int t_end = min(t_begin + a.part_tokens, ctx);
    const int n_parts = (ctx + a.part_tokens - 1) / a.part_tokens;

    cl_f4 q[NV], o[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        q[j] = *reinterpret_cast<const cl_f4 *>(a.q + head_off + 64 * j + 4 * c16);
        o[j] = (cl_f4){0.f, 0.f, 0.f, 0.f};
    }
    const int32_t *bt = a.block_tables + (size_t)b * a.max_blocks;
    const size_t row_stride = (size_t)H * D;  // floats between consecutive slots
    const size_t lane_off = (size_t)h * D + 4 * c16 + (size_t)row * row_stride;
    const size_t new_off = head_off + 4 * c16;
    WaveState st{-INFINITY, 0.0f};

    const int lb_first = t_begin / BS, lb_last = (t_end - 1) / BS;
    const bool tail_checked = t_end == ctx && (ctx % BS != 0 || a.k_new != nullptr);
    for (int lb = lb_first + wave; lb <= lb_last; lb += 4) {
        const int64_t blk = bt[lb];
        if (blk < 0 || blk >= a.num_blocks) {
            if (lane == 0) atomicOr(a.err_flag, 1);
            continue;
        }
        const size_t off = (size_t)blk * BS * row_stride + lane_off;
        if (tail_checked && lb == lb_last)
            fold_block<D, BS, true>(a, a.k_cache + off, a.v_cache + off, row_stride, lb * BS,
                                    t_end, ctx, row, new_off, q, st, o);
        else
            fold_block<D, BS, false>(a, a.k_cache + off, a.v_cache + off, row_stride, lb * BS,
                                     t_end, ctx, row, new_off, q, st, o);
    }

    // Merge the four token rows of the wave (same running max everywhere).
    st.l += __shfl_xor(st.l, 16, 64);
    st.l += __shfl_xor(st.l, 32, 64);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            float v = o[j][c];
            v += __shfl_xor(v, 16, 64);
            v += __shfl_xor(v, 32, 64);
            o[j][c] = v;
        }
    }
    if (row == 0) {
#pragma unroll
        for (int j = 0; j < NV; ++j) *reinterpret_cast<cl_f4 *>(&s_o[wave][64 * j + 4 * c16]) = o[j];
    }
    if (lane == 0) {
        s_m[wave] = st.m;
        s_l[wave] = st.l;
    }
    __syncthreads();

    // Merge the four waves: thread d < D owns output element d.
    const int d = threadIdx.x;
    float M = -INFINITY, L = 0.0f, O = 0.0f;
    if (d < D) {
#pragma unroll
        for (int w = 0; w < 4; ++w) M = fmaxf(M, s_m[w]);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            if (s_m[w] == -INFINITY) continue;
            const float e = fast_exp(s_m[w] - M);
            L += s_l[w] * e;
            O += s_o[w][d] * e;
        }
    }
    if (n_parts == 1) {
        if (d < D) a.out[head_off + d] = O / L;
        return;
    }
    float *ws = a.partials + ((size_t)b * H + h) * a.max_parts * (D + 2);
    if (d < D) {
        ws[part * (D + 2) + d] = O;
        if (d == 0) {
            ws[part * (D + 2) + D] = M;
            ws[part * (D + 2) + D + 1] = L;
        }
    }
    // Last workgroup of this (b, h) merges every partition.
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        const int ticket = atomicAdd(a.counters + (size_t)b * H + h, 1);
        s_last = ticket == n_parts - 1;
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    if (d < D) {
        float gm = -INFINITY;
        for (int p = 0; p < n_parts; ++p) gm = fmaxf(gm, ws[p * (D + 2) + D]);
        float gl = 0.0f, go = 0.0f;
        for (int p = 0; p < n_parts; ++p) {
            const float mp = ws[p * (D + 2) + D];
            if (mp == -INFINITY) continue;
            const float e = fast_exp(mp - gm);
            gl += ws[p * (D + 2) + D + 1] * e;
            go += ws[p * (D + 2) + d] * e;
        }
        a.out[head_off + d] = go / gl;
    }
    if (threadIdx.x == 0) a.counters[(size_t)b * H + h] = 0;
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
