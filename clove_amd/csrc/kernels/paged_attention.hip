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
// workgroup handles one partition of one sequence for four adjacent heads,
// one wave per head.  Measured on MI355X at the benchmark shape
// (B=32, H=32, D=128, ctx 512..4096): head-major waves with 2048-token
// partitions stream at ~6 TB/s, against ~5.1 TB/s when the four waves split
// one head's KV blocks (each workgroup then reads 512-byte rows at a 16 KiB
// stride while the neighbouring heads of the same tokens are read at
// unrelated times).
//
// Lane layout.  A token's head row (D floats, contiguous) belongs to one
// 16-lane DPP row of the wave: lane c of the row holds the 16-byte pieces
// at floats 4c, 64+4c, ... (D/64 pieces).  One wave load therefore reads
// four whole token rows in 256-byte contiguous runs, every byte fetched is
// used, and q.k is reduced inside the DPP row with four full-rate
// v_add_f32_dpp (quad_perm 1032, quad_perm 2301, row_ror 4, row_ror 8) --
// no LDS traffic.  A KV block (16 tokens) is 4 such loads for K and 4 for
// V per piece.  Only the block that holds token ctx-1 can be partial or
// carry the new token; it alone takes the per-token checked path.
//
// Streaming.  Whole blocks go through a two-deep register pipeline: block
// n + 1's K and V loads are issued before block n is folded, so a wave
// keeps up to two blocks (32 KiB at D=128, BS=16) in flight and never waits
// for more than the older one.  The partition's table entries are read into
// registers once, up front (which also validates them), so no table load
// sits between KV loads in the in-order vmcnt queue.  K and V are loaded
// non-temporally: each row is read once per launch.  Measured at the
// benchmark shape: 76.7% of HBM peak with plain loads and one block in
// flight, 80.8% with non-temporal loads, 82.0% with the pipeline.
//
// Softmax.  Each wave keeps a running (max, sum, acc) (online softmax); a
// partition's (max, sum, acc) goes to a workspace that a one-wave-per-(b, h)
// kernel merges with the log-sum-exp rule (a device-wide fence plus ticket
// inside the partition kernel would write back the per-XCD L2s and costs
// far more than the second launch).
// exp is the hardware 2^x of x*log2(e) (relative error ~1e-6, far below the
// 2e-3 parity bound).
//
// Safety: context lengths are clamped to the table's capacity and table
// entries outside [0, num_blocks) are skipped; both set a device error flag
// that the host reports at its next synchronisation point.  No load is ever
// issued outside the pool.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdlib>

#include "launch.hpp"
#include "wave.h"

namespace clove {
namespace k {

namespace {

__device__ __forceinline__ int clamp_ctx(const PagedArgs &a, int b, bool report) {
    int ctx = a.context_lens[b];
    const int cap = a.max_blocks * a.block_size;
    if (ctx < 0 || ctx > cap) {
        if (report) atomicOr(a.err_flag, kErrPagedRange);
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

// K and V rows are read exactly once per launch: non-temporal loads keep
// them from displacing other lines in L2.  On MI355X this raised a
// loads-only stream over the benchmark's 2.35 GB of KV rows from 74% to 78%
// of HBM peak.
__device__ __forceinline__ cl_f4 stream_load(const float *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const cl_f4 *>(p));
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
                kk[s][j] = stream_load(kp + 64 * j);
                vv[s][j] = stream_load(vp + 64 * j);
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

// The K and V rows of one whole KV block as this lane holds them: step s
// covers rows 4s + (lane >> 4), piece j floats 64j + 4(lane & 15).
template <int D, int BS>
struct BlockRegs {
    cl_f4 k[BS / 4][D / 64], v[BS / 4][D / 64];
};

// Issues every K and V load of one whole block (`off` = this lane's offset
// of the block's row `row` in a plane) without waiting for any of them.
template <int D, int BS>
__device__ __forceinline__ void issue_block(const PagedArgs &a, size_t off, size_t row_stride,
                                            BlockRegs<D, BS> &r) {
#pragma unroll
    for (int s = 0; s < BS / 4; ++s)
#pragma unroll
        for (int j = 0; j < D / 64; ++j) {
            r.k[s][j] = stream_load(a.k_cache + off + (size_t)(4 * s) * row_stride + 64 * j);
            r.v[s][j] = stream_load(a.v_cache + off + (size_t)(4 * s) * row_stride + 64 * j);
        }
}

// Folds a block whose loads `issue_block` issued into the running state
// (the arithmetic of fold_block without the per-token checks).
template <int D, int BS>
__device__ __forceinline__ void consume_block(const PagedArgs &a, const BlockRegs<D, BS> &r,
                                              const cl_f4 (&q)[D / 64], WaveState &st,
                                              cl_f4 (&o)[D / 64]) {
    constexpr int NV = D / 64;
    constexpr int T = BS / 4;
    float sc[T];
    float bm = -INFINITY;
#pragma unroll
    for (int s = 0; s < T; ++s) {
        float d = dot4(q[0], r.k[s][0]);
#pragma unroll
        for (int j = 1; j < NV; ++j) d += dot4(q[j], r.k[s][j]);
        sc[s] = row16_sum(d) * a.scale;
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
    for (int s = 0; s < T; ++s) {
        const float p = fast_exp(sc[s] - m_new);
        st.l += p;
#pragma unroll
        for (int j = 0; j < NV; ++j) o[j] += p * r.v[s][j];
    }
    st.m = m_new;
}

// Table entries of a partition held in registers: entry i (relative to the
// partition's first whole block) is lane i % 64 of tab[i / 64].  Reading
// them with readlane keeps vector loads of the table out of the block loop,
// where the in-order vmcnt counter would make each wait for a table entry
// also wait for the KV loads issued before it.
constexpr int kTabRegs = 4;

__device__ __forceinline__ int64_t table_entry(const int (&tab)[kTabRegs], int i) {
    const int r = i >> 6;
    const int v = r == 0 ? tab[0] : r == 1 ? tab[1] : r == 2 ? tab[2] : tab[3];
    return __builtin_amdgcn_readlane(v, i & 63);
}

// Folds `n` whole blocks (n <= 64 * kTabRegs) whose table entries `tab`
// holds, all inside the pool, two register buffers deep: sub-block i + 1's
// loads are in flight while sub-block i is folded.  A block of BS tokens is
// folded as BS / SB sub-blocks of SB consecutive tokens (rows), each one
// step of the online softmax.  Every load is unconditional, so the wait
// before each fold only drains the older buffer.
template <int D, int BS, int SB>
__device__ __forceinline__ void fold_pipelined(const PagedArgs &a, const int (&tab)[kTabRegs],
                                               int n, size_t lane_off, size_t row_stride,
                                               const cl_f4 (&q)[D / 64], WaveState &st,
                                               cl_f4 (&o)[D / 64]) {
    constexpr int NS = BS / SB;
    const size_t blk_stride = (size_t)BS * row_stride;
    auto sub_off = [&](int j) {  // sub-block j of the partition's whole blocks
        return (size_t)table_entry(tab, j / NS) * blk_stride + lane_off +
               (size_t)((j % NS) * SB) * row_stride;
    };
    const int subs = n * NS;
    BlockRegs<D, SB> A, B;
    int i = 0;
    issue_block<D, SB>(a, sub_off(0), row_stride, A);
    for (; i + 2 < subs; i += 2) {
        issue_block<D, SB>(a, sub_off(i + 1), row_stride, B);
        consume_block<D, SB>(a, A, q, st, o);
        issue_block<D, SB>(a, sub_off(i + 2), row_stride, A);
        consume_block<D, SB>(a, B, q, st, o);
    }
    if (i + 1 < subs) {
        issue_block<D, SB>(a, sub_off(i + 1), row_stride, B);
        consume_block<D, SB>(a, A, q, st, o);
        consume_block<D, SB>(a, B, q, st, o);
    } else {
        consume_block<D, SB>(a, A, q, st, o);
    }
}

// One workgroup = HPW adjacent heads of one (partition, sequence); wave w
// owns head HPW*blockIdx.x + w for the whole partition.  The waves walk the
// same KV blocks together, so a token's HPW head rows (HPW * D * 4 bytes,
// contiguous in the pool) are read at the same time, and the grid's fastest
// dimension is the head group, so neighbouring workgroups read the other
// heads of the same tokens: the pool is streamed in long contiguous runs.
template <int D, int BS, int HPW>
__global__ void __launch_bounds__(64 * HPW) paged_heads_kernel(PagedArgs a) {
    constexpr int NV = D / 64;
    // Tokens per online-softmax step.  A whole block at head_dim 256 and 32
    // tokens is 512 floats of K and V per lane, two of them twice that: the
    // pipeline spilled to scratch (5.5 against 6.2 TB/s with 16-token
    // blocks).  There the block is folded as two 16-token halves, in every
    // path alike, so all paths still round the same way.
    constexpr int SB = (D >= 256 && BS >= 32) ? BS / 2 : BS;
    constexpr int NS = BS / SB;
    const int part = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int h = blockIdx.x * HPW + wave;
    const int H = a.num_heads;
    if (h >= H) return;
    const int row = lane >> 4, c16 = lane & 15;
    const size_t head_off = ((size_t)b * H + h) * D;
    const int ctx = clamp_ctx(a, b, part == 0 && h == 0 && lane == 0);
    const int t_begin = part * a.part_tokens;
    if (t_begin >= ctx) {
        if (ctx == 0 && part == 0) {
            for (int d = lane; d < D; d += 64) a.out[head_off + d] = 0.0f;
        }
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
    const size_t row_stride = (size_t)H * D;
    const size_t lane_off = (size_t)h * D + 4 * c16 + (size_t)row * row_stride;
    const size_t new_off = head_off + 4 * c16;
    WaveState st{-INFINITY, 0.0f};

    const int lb_first = t_begin / BS, lb_last = (t_end - 1) / BS;
    const bool tail_checked = t_end == ctx && (ctx % BS != 0 || a.k_new != nullptr);
    const int64_t nb = a.num_blocks;
    const int full_end = tail_checked ? lb_last : lb_last + 1;  // whole blocks: [lb_first, full_end)
    // Whole blocks: the pipelined fold when the range has at most
    // 64 * kTabRegs blocks and every table entry is inside the pool (checked
    // by the wave up front), else block by block with bad entries skipped
    // and reported.
    const int n_full = full_end - lb_first;
    int tab[kTabRegs];
    bool bad = false;
#pragma unroll
    for (int r = 0; r < kTabRegs; ++r) {
        const int i = lb_first + 64 * r + lane;
        tab[r] = i < full_end ? bt[i] : 0;
        bad = bad || tab[r] < 0 || tab[r] >= nb;
    }
    if (n_full > 0 && n_full <= 64 * kTabRegs && !__any(bad)) {
        fold_pipelined<D, BS, SB>(a, tab, n_full, lane_off, row_stride, q, st, o);
    } else {
        for (int lb = lb_first; lb < full_end; ++lb) {
            const int64_t blk = bt[lb];
            if (blk < 0 || blk >= nb) {
                if (lane == 0) atomicOr(a.err_flag, kErrPagedRange);
                continue;
            }
#pragma unroll
            for (int sb = 0; sb < NS; ++sb) {
                BlockRegs<D, SB> r;
                issue_block<D, SB>(a, (size_t)(blk * BS + sb * SB) * row_stride + lane_off,
                                   row_stride, r);
                consume_block<D, SB>(a, r, q, st, o);
            }
        }
    }
    if (tail_checked) {
        const int64_t blk = bt[lb_last];
        if (blk < 0 || blk >= nb) {
            if (lane == 0) atomicOr(a.err_flag, kErrPagedRange);
        } else {
            const size_t off = (size_t)blk * BS * row_stride + lane_off;
#pragma unroll
            for (int sb = 0; sb < NS; ++sb) {
                const size_t so = off + (size_t)(sb * SB) * row_stride;
                fold_block<D, SB, true>(a, a.k_cache + so, a.v_cache + so, row_stride,
                                        lb_last * BS + sb * SB, t_end, ctx, row, new_off, q, st,
                                        o);
            }
        }
    }
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
    if (row != 0) return;
    if (n_parts == 1) {
        const float inv = 1.0f / st.l;
#pragma unroll
        for (int j = 0; j < NV; ++j)
            *reinterpret_cast<cl_f4 *>(a.out + head_off + 64 * j + 4 * c16) = o[j] * inv;
        return;
    }
    float *ws = a.partials + (((size_t)b * H + h) * a.max_parts + part) * (D + 2);
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int c = 0; c < 4; ++c) ws[64 * j + 4 * c16 + c] = o[j][c];
    if (c16 == 0) {
        ws[D] = st.m;
        ws[D + 1] = st.l;
    }
}

// ---- General decode: any head_dim up to 1024, any block size ----------------
//
// The kernel above fixes head_dim and block size at compile time and reads
// whole KV blocks per load step.  Clove's modules give head_dim = dim /
// num_heads with no restriction (nn.rs:519, nn/attention.rs:47) and the lazy
// plan takes it from q's last dimension (lazy.rs:2363-2371), so every other
// shape runs here:
//   * a token's head row (D floats) belongs to a group of L = 8 or 16
//     adjacent lanes, so one wave load covers 64 / L tokens.  Lane c of a
//     group holds NP pieces of four floats: piece j is floats 4Lj + 4c ..
//     4Lj + 4c + 3 when D % 4 == 0 (one 16-byte load, VEC4), floats
//     4Lj + c + L*e, e = 0..3, otherwise (four 4-byte loads).  (L, NP) is
//     chosen per head dim to leave the fewest lanes idle (D = 96: L = 8,
//     NP = 3, none idle); floats at or past D read as zero, so q . k and the
//     output need no other mask.  q . k is summed over the group with DPP.
//   * the workgroup's four waves (four heads of one sequence) walk the same
//     tokens and share one LDS table of their physical rows, built kGenChunk
//     tokens at a time from the block table (row = bt[t / bs] * bs + t % bs),
//     so any block size costs one LDS read per token and partitions need not
//     align with blocks.  The new token (t = ctx - 1 with k/v given) and
//     tokens past the range or behind a bad table entry are marked in it.
//   * tokens are folded TS * 64 / L at a time (one online-softmax step of the
//     arithmetic of fold_block), two register buffers deep while both fit
//     (NP <= 8, D <= 512), one buffer beyond.
// A lane with no token loads the pool's first row (always inside it) and its
// values are replaced by zero, so no load is conditional; a piece that can
// reach past D (the last, or any when NP >= 8) has its address checked per
// lane.
constexpr int kGenChunk = 512;
constexpr int kRowNone = -1;  // no token: past the range, or a bad table entry
constexpr int kRowNew = -2;   // token ctx - 1 taken from k_new / v_new

template <int L, int NP>
struct GenShape {
    static constexpr int T = 64 / L;  // tokens per wave load
    // 4-token steps per fold: at most 64 floats of K and V per buffer and lane,
    // at most 32 tokens per online-softmax step
    static constexpr int TS0 = 8 / NP < 1 ? 1 : 8 / NP;
    static constexpr int TS = TS0 * T > 32 ? 32 / T : TS0;
    static constexpr bool PIPE = NP <= 8;
};

template <int L, int NP>
struct GenRegs {
    cl_f4 k[GenShape<L, NP>::TS][NP], v[GenShape<L, NP>::TS][NP];
    bool in[GenShape<L, NP>::TS];
};

// Float index of piece j, component e, in lane c of its group.
template <int L, bool VEC4>
__device__ __forceinline__ int gen_float(int j, int e, int c) {
    return VEC4 ? 4 * L * j + 4 * c + e : 4 * L * j + c + L * e;
}

// Loads the NP pieces of the row at `row` (null: no token) into `out`.
// `shift` floats (a multiple of 4, VEC4 only) move the pieces back so that
// they start on a 128-byte line (see paged_general_kernel): float f of the
// row is then in piece slot f + shift.
template <int L, int NP, bool VEC4>
__device__ __forceinline__ void gen_row(const float *row, const float *safe, int c, int D,
                                        int shift, cl_f4 (&out)[NP]) {
    const float *base = row ? row : safe;
#pragma unroll
    for (int j = 0; j < NP; ++j) {
        // Unshifted with NP < 8, general_plan picks (L, NP) only for head
        // dims that leave fewer than L idle piece slots, so the pieces
        // before the last are inside the row and only the last may pass D;
        // shifted, or with NP >= 8, any piece can be outside, and every
        // piece is checked.
        const bool last = NP >= 8 || shift != 0 || j == NP - 1;
        if (VEC4) {
            const int f = gen_float<L, true>(j, 0, c) - shift;
            const bool use = !last || (f >= 0 && f < D);
            const cl_f4 v = stream_load(use ? base + f : base);
            out[j] = (row && use) ? v : (cl_f4){0.f, 0.f, 0.f, 0.f};
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int f = gen_float<L, false>(j, e, c);
                const bool use = !last || f < D;
                const float v = __builtin_nontemporal_load(use ? base + f : base);
                out[j][e] = (row && use) ? v : 0.0f;
            }
        }
    }
}

// Sum over the L lanes of a group (every lane of the group gets it).
template <int L>
__device__ __forceinline__ float group_sum(float v) {
    v += dpp<0xB1>(v);  // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);  // quad_perm [2,3,0,1]
    if (L >= 8) v += dpp<0x141>(v);   // row_half_mirror: quad q + quad q^1
    if (L >= 16) v += dpp<0x140>(v);  // row_mirror: half h + half h^1
    return v;
}

// Combines the token groups of the wave: every lane gets the max / sum over
// the lanes with its index within the group.
template <int L>
__device__ __forceinline__ float groups_max(float v) {
    if (L <= 4) v = fmaxf(v, dpp<0x124>(v));  // row_ror 4
    if (L <= 8) v = fmaxf(v, dpp<0x128>(v));  // row_ror 8
    v = fmaxf(v, __shfl_xor(v, 16, 64));
    return fmaxf(v, __shfl_xor(v, 32, 64));
}
template <int L>
__device__ __forceinline__ float groups_sum(float v) {
    if (L <= 4) v += dpp<0x124>(v);
    if (L <= 8) v += dpp<0x128>(v);
    v += __shfl_xor(v, 16, 64);
    return v + __shfl_xor(v, 32, 64);
}

// HP = 2 (head pairs, D = 16 and 48 with H even): a group's row is the 2D
// floats of heads 2p and 2p + 1, which start on a 128-byte line for every
// token; L = 8 lanes take D / 16 pieces each, none idle, and no load touches
// a line that another wave also reads.  Each piece belongs to one head of the
// pair (pieces hold four floats and D % 4 == 0), so q . k, the online
// softmax and the output are kept per head.  At the config-5 shape: D = 16
// 38.2 -> 45.7%, D = 48 56.9 -> 61.6% of HBM.  D = 80 and 112 (five and seven
// pieces per lane) fold 8 tokens per softmax step against 16 for the single
// heads, twice the softmax work per token, and measured slower (48.6 / 58.7%
// against 57.6 / 65.4%; 56.4% at D = 80 folding 16 tokens in 256 VGPRs).
template <int L, int NP, bool VEC4, int HP = 1>
__global__ void __launch_bounds__(256) paged_general_kernel(PagedArgs a) {
    static_assert(HP == 1 || (HP == 2 && VEC4), "head pairs move 16-byte pieces");
    using Sh = GenShape<L, NP>;
    using Regs = GenRegs<L, NP>;
    constexpr int T = Sh::T, TS = Sh::TS;
    __shared__ int rows_lds[kGenChunk];
    const int part = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int H = a.num_heads, D = a.head_dim, BS = a.block_size;
    const int DR = HP * D;                   // floats of the row a group reads
    const int h = HP * (blockIdx.x * 4 + wave);  // the row's first head
    const bool active = h < H;  // idle waves still take part in the barriers
    // With a.gen_shift (H * D a multiple of 32 floats, so head h's rows sit
    // at the same offset in their 128-byte lines for every token), the
    // wave's pieces start at the line boundary before its rows: each wave
    // load then touches whole lines, where a row that starts mid-line (D =
    // 48, 80, 112) makes every load touch twice the lines.  q and the output
    // use the same float-to-lane map.  (Head pairs start on a line.)
    const int shift = HP == 1 && VEC4 && a.gen_shift ? (h * D) % 32 : 0;
    const int grp = lane / L, c = lane % L;
    const size_t head_off = ((size_t)b * H + (active ? h : 0)) * D;
    const int ctx = clamp_ctx(a, b, part == 0 && threadIdx.x == 0);
    const int t_begin = part * a.part_tokens;
    if (t_begin >= ctx) {  // uniform over the workgroup
        if (ctx == 0 && part == 0 && active)
            for (int d = lane; d < DR; d += 64) a.out[head_off + d] = 0.0f;
        return;
    }
    const int t_end = min(t_begin + a.part_tokens, ctx);
    const int n_parts = (ctx + a.part_tokens - 1) / a.part_tokens;
    const int32_t *bt = a.block_tables + (size_t)b * a.max_blocks;
    const size_t row_stride = (size_t)H * D;
    const size_t h_off = (size_t)(active ? h : 0) * D;

    cl_f4 q[NP], o[NP];
    gen_row<L, NP, VEC4>(active ? a.q + head_off : nullptr, a.q, c, DR, shift, q);
#pragma unroll
    for (int j = 0; j < NP; ++j) o[j] = (cl_f4){0.f, 0.f, 0.f, 0.f};
    WaveState st[HP];
#pragma unroll
    for (int u = 0; u < HP; ++u) st[u] = WaveState{-INFINITY, 0.0f};
    bool second[NP];  // piece j of this lane belongs to the pair's second head
#pragma unroll
    for (int j = 0; j < NP; ++j) second[j] = HP == 2 && gen_float<L, VEC4>(j, 0, c) >= D;

    auto issue = [&](int t0, int cb, int ce, Regs &r) {
#pragma unroll
        for (int s = 0; s < TS; ++s) {
            const int t = t0 + T * s + grp;
            const int rw = t < ce ? rows_lds[t - cb] : kRowNone;
            r.in[s] = rw != kRowNone;
            const float *kp = nullptr, *vp = nullptr;
            if (rw == kRowNew) {
                kp = a.k_new + head_off;
                vp = a.v_new + head_off;
            } else if (rw >= 0) {
                const size_t off = (size_t)rw * row_stride + h_off;
                kp = a.k_cache + off;
                vp = a.v_cache + off;
            }
            gen_row<L, NP, VEC4>(kp, a.k_cache, c, DR, shift, r.k[s]);
            gen_row<L, NP, VEC4>(vp, a.k_cache, c, DR, shift, r.v[s]);
        }
    };
    auto consume = [&](const Regs &r) {
        float sc[HP][TS];
        float bm[HP];
#pragma unroll
        for (int u = 0; u < HP; ++u) bm[u] = -INFINITY;
#pragma unroll
        for (int s = 0; s < TS; ++s) {
            float d[HP];
            if constexpr (HP == 1) {
                d[0] = dot4(q[0], r.k[s][0]);
#pragma unroll
                for (int j = 1; j < NP; ++j) d[0] += dot4(q[j], r.k[s][j]);
            } else {
                d[0] = d[1] = 0.0f;
#pragma unroll
                for (int j = 0; j < NP; ++j) {
                    const float t = dot4(q[j], r.k[s][j]);
                    d[0] += second[j] ? 0.0f : t;
                    d[1] += second[j] ? t : 0.0f;
                }
            }
#pragma unroll
            for (int u = 0; u < HP; ++u) {
                d[u] = group_sum<L>(d[u]);
                sc[u][s] = r.in[s] ? d[u] * a.scale : -INFINITY;
                bm[u] = fmaxf(bm[u], sc[u][s]);
            }
        }
        float m_new[HP], alpha[HP];
#pragma unroll
        for (int u = 0; u < HP; ++u) {
            bm[u] = groups_max<L>(bm[u]);
            m_new[u] = fmaxf(st[u].m, bm[u]);
            alpha[u] = (st[u].m == -INFINITY) ? 0.0f : fast_exp(st[u].m - m_new[u]);
            st[u].l *= alpha[u];
        }
#pragma unroll
        for (int j = 0; j < NP; ++j) o[j] *= HP == 2 && second[j] ? alpha[HP - 1] : alpha[0];
#pragma unroll
        for (int s = 0; s < TS; ++s) {
            float p[HP];
#pragma unroll
            for (int u = 0; u < HP; ++u) {
                p[u] = r.in[s] ? fast_exp(sc[u][s] - m_new[u]) : 0.0f;
                st[u].l += p[u];
            }
#pragma unroll
            for (int j = 0; j < NP; ++j) o[j] += (HP == 2 && second[j] ? p[HP - 1] : p[0]) * r.v[s][j];
        }
#pragma unroll
        for (int u = 0; u < HP; ++u) st[u].m = m_new[u];
    };

    const int64_t nb = a.num_blocks;
    for (int cb = t_begin; cb < t_end; cb += kGenChunk) {
        const int ce = min(cb + kGenChunk, t_end);
        __syncthreads();  // every wave is done with the previous chunk's rows
        for (int i = threadIdx.x; i < ce - cb; i += 256) {
            const int t = cb + i;
            int rw = kRowNone;
            if (a.k_new != nullptr && t == ctx - 1) {
                rw = kRowNew;
            } else {
                const int lb = t / BS;
                const int64_t e = bt[lb];
                if (e >= 0 && e < nb) {
                    rw = (int)(e * BS + (t - lb * BS));
                } else if (i == 0 || t - lb * BS == 0) {
                    atomicOr(a.err_flag, kErrPagedRange);
                }
            }
            rows_lds[i] = rw;
        }
        __syncthreads();
        if (!active) continue;
        constexpr int G = T * TS;  // tokens per fold
        if (Sh::PIPE) {
            Regs A, B;
            int t0 = cb;
            issue(t0, cb, ce, A);
            for (; t0 + 2 * G < ce; t0 += 2 * G) {
                issue(t0 + G, cb, ce, B);
                consume(A);
                issue(t0 + 2 * G, cb, ce, A);
                consume(B);
            }
            if (t0 + G < ce) {
                issue(t0 + G, cb, ce, B);
                consume(A);
                consume(B);
            } else {
                consume(A);
            }
        } else {
            for (int t0 = cb; t0 < ce; t0 += G) {
                Regs A;
                issue(t0, cb, ce, A);
                consume(A);
            }
        }
    }
    if (!active) return;
#pragma unroll
    for (int u = 0; u < HP; ++u) st[u].l = groups_sum<L>(st[u].l);
#pragma unroll
    for (int j = 0; j < NP; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) o[j][e] = groups_sum<L>(o[j][e]);
    if (grp != 0) return;
    // float f of the row: head h + f / D, dim f % D (a piece never straddles)
    if (n_parts == 1) {
        float inv[HP];
#pragma unroll
        for (int u = 0; u < HP; ++u) inv[u] = 1.0f / st[u].l;
#pragma unroll
        for (int j = 0; j < NP; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int f = gen_float<L, VEC4>(j, e, c) - shift;
                if (f >= 0 && f < DR)
                    a.out[head_off + f] = o[j][e] * (HP == 2 && second[j] ? inv[HP - 1] : inv[0]);
            }
        return;
    }
    float *ws[HP];
#pragma unroll
    for (int u = 0; u < HP; ++u)
        ws[u] = a.partials + (((size_t)b * H + h + u) * a.max_parts + part) * (D + 2);
#pragma unroll
    for (int j = 0; j < NP; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int f = gen_float<L, VEC4>(j, e, c) - shift;
            if (f >= 0 && f < DR) {
                if (HP == 2 && second[j]) ws[HP - 1][f - D] = o[j][e];
                else ws[0][f] = o[j][e];
            }
        }
    if (c == 0) {
#pragma unroll
        for (int u = 0; u < HP; ++u) {
            ws[u][D] = st[u].m;
            ws[u][D + 1] = st[u].l;
        }
    }
}

// Merges the partitions of each (b, h) with the log-sum-exp rule:
// out = sum_p O_p e^(M_p - M) / sum_p L_p e^(M_p - M).  One wave per (b, h);
// sequences that fit one partition were written by the partition kernel.
__global__ void __launch_bounds__(256) paged_merge_kernel(PagedArgs a) {
    const int lane = threadIdx.x & 63;
    const int pair = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (pair >= a.num_seqs * a.num_heads) return;
    const int b = pair / a.num_heads;
    const int D = a.head_dim;
    const int ctx = clamp_ctx(a, b, false);
    const int n_parts = (ctx + a.part_tokens - 1) / a.part_tokens;
    if (n_parts <= 1) return;
    const float *ws = a.partials + (size_t)pair * a.max_parts * (D + 2);
    float M = -INFINITY;
#pragma unroll 8
    for (int p = 0; p < n_parts; ++p) M = fmaxf(M, ws[p * (D + 2) + D]);
    float L = 0.0f;
#pragma unroll 8
    for (int p = 0; p < n_parts; ++p) {
        const float mp = ws[p * (D + 2) + D];
        L += mp == -INFINITY ? 0.0f : ws[p * (D + 2) + D + 1] * fast_exp(mp - M);
    }
    const float invL = 1.0f / L;
    for (int d = lane; d < D; d += 64) {
        float O = 0.0f;
#pragma unroll 8
        for (int p = 0; p < n_parts; ++p) {
            const float mp = ws[p * (D + 2) + D];
            O += mp == -INFINITY ? 0.0f : ws[p * (D + 2) + d] * fast_exp(mp - M);
        }
        a.out[(size_t)pair * D + d] = O * invL;
    }
}

// Writes the new token's K and V rows of every sequence into its cache slot.
// One workgroup per sequence copies H*D floats per plane as 16-byte vectors.
__global__ void __launch_bounds__(256) paged_append_kernel(float *__restrict__ k_cache,
                                                           float *__restrict__ v_cache,
                                                           const float *__restrict__ k_new,
                                                           const float *__restrict__ v_new,
                                                           const int32_t *__restrict__ bt,
                                                           const int32_t *__restrict__ cl,
                                                           int max_blocks, int bs, int64_t num_blocks,
                                                           int row_floats, int32_t *err_flag) {
    const int b = blockIdx.x;
    const int ctx = cl[b];
    if (ctx <= 0) return;
    if (ctx > max_blocks * bs) {
        if (threadIdx.x == 0) atomicOr(err_flag, kErrPagedRange);
        return;
    }
    const int64_t blk = bt[(size_t)b * max_blocks + (ctx - 1) / bs];
    if (blk < 0 || blk >= num_blocks) {
        if (threadIdx.x == 0) atomicOr(err_flag, kErrPagedRange);
        return;
    }
    const size_t dst = ((size_t)blk * bs + (ctx - 1) % bs) * row_floats;
    const size_t src = (size_t)b * row_floats;
    for (int i = threadIdx.x; i < row_floats / 4; i += 256) {
        reinterpret_cast<cl_f4 *>(k_cache + dst)[i] = reinterpret_cast<const cl_f4 *>(k_new + src)[i];
        reinterpret_cast<cl_f4 *>(v_cache + dst)[i] = reinterpret_cast<const cl_f4 *>(v_new + src)[i];
    }
}

__global__ void __launch_bounds__(256) paged_slots_kernel(const int32_t *__restrict__ bt,
                                                          const int32_t *__restrict__ cl,
                                                          int32_t *__restrict__ slots,
                                                          int num_seqs, int max_blocks, int bs,
                                                          int max_ctx, int32_t *err_flag) {
    const int64_t total = (int64_t)num_seqs * max_ctx;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * 256) {
        const int b = (int)(i / max_ctx), t = (int)(i % max_ctx);
        const int ctx = cl[b];
        int32_t slot = -1;
        if (t < ctx && t < max_blocks * bs) {
            const int32_t e = bt[(size_t)b * max_blocks + t / bs];
            // every slot of block e must be a non-negative int32
            if (e >= 0 && (int64_t)e * bs + bs <= (int64_t)INT32_MAX)
                slot = e * bs + t % bs;
            else
                atomicOr(err_flag, kErrPagedRange);
        }
        slots[i] = slot;
    }
}

// An f32 index value: v when v is an integer in [0, 2^24) (f32 represents
// all of them exactly, so the comparison with its truncation and the
// conversion are exact), else -1.
__device__ __forceinline__ int32_t index_value(float v) {
    return (v >= 0.0f && v < 16777216.0f && v == truncf(v)) ? (int32_t)v : -1;
}

__global__ void __launch_bounds__(256) paged_index_kernel(const float *__restrict__ bt_f,
                                                          int32_t *__restrict__ bt_out,
                                                          const float *__restrict__ cl_f,
                                                          const int32_t *__restrict__ cl_i,
                                                          int32_t *__restrict__ cl_out,
                                                          int num_seqs, int max_blocks, int bs,
                                                          int32_t *err_flag) {
    const int64_t n_bt = bt_f ? (int64_t)num_seqs * max_blocks : 0;
    const int64_t n_cl = cl_f ? num_seqs : 0;
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n_cl + n_bt; i += stride) {
        if (i < n_cl) {
            const int32_t c = index_value(cl_f[i]);
            if (c < 0) atomicOr(err_flag, kErrIndexValue);
            cl_out[i] = c;
            continue;
        }
        const int64_t e = i - n_cl;
        const int b = (int)(e / max_blocks), j = (int)(e % max_blocks);
        const int32_t ctx = cl_f ? index_value(cl_f[b]) : cl_i[b];
        const int32_t v = index_value(bt_f[e]);
        if (v < 0 && ctx > 0 && (int64_t)j * bs < (int64_t)ctx) atomicOr(err_flag, kErrIndexValue);
        bt_out[e] = v;
    }
}

// Partition workspace of the allocation-free decode entry
// (clove_hip_paged_attention_noalloc): one array per GPU, alive until the
// process ends.  Host code never names it in a launch or a copy: it takes
// the device address once per device (paged_scratch_address) and passes that.
// Every partial a launch's merge reads is written by the same launch's
// partition kernel first, so nothing in it needs clearing.
static __device__ __align__(256) float scratch[kPagedScratchFloats];

}  // namespace

hipError_t paged_scratch_address(float **ptr) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    *ptr = e == hipSuccess ? static_cast<float *>(p) : nullptr;
    return e;
}

// Shapes the fixed-shape kernel (paged_heads_kernel) is built for.
static bool paged_tuned(int head_dim, int block_size) {
    return (head_dim == 64 || head_dim == 128 || head_dim == 256) &&
           (block_size == 8 || block_size == 16 || block_size == 32);
}

bool paged_supported(int head_dim, int block_size) {
    return head_dim >= 1 && head_dim <= kPagedMaxHeadDim && block_size >= 1;
}

// Partition length: long partitions stream best, but the grid should still
// hold about two workgroups per CU when every context is full; the result
// is a power of two between 256 and 2048 tokens, rounded to whole KV
// blocks.  CLOVE_PAGED_PART overrides it (tuning only; the output does not
// depend on it beyond summation order).
int paged_part_tokens(int num_seqs, int num_heads, int capacity, int block_size, int num_cus) {
    int tokens;
    const char *v = std::getenv("CLOVE_PAGED_PART");
    if (v && *v) {
        tokens = std::atoi(v);
    } else {
        const int64_t groups = (int64_t)num_seqs * ((num_heads + 3) / 4);
        const int64_t want = 2LL * num_cus;
        tokens = 256;
        while (tokens < 2048 && groups * ((capacity + 2 * tokens - 1) / (2 * tokens)) >= want)
            tokens *= 2;
    }
    int blocks = tokens / block_size;
    if (blocks < 1) blocks = 1;
    return blocks * block_size;
}

size_t paged_workspace_floats(int num_seqs, int num_heads, int head_dim, int max_ctx,
                              int part_tokens) {
    const int parts = (max_ctx + part_tokens - 1) / part_tokens;
    if (parts <= 1) return 0;
    return (size_t)num_seqs * num_heads * parts * (head_dim + 2);
}

// The general kernel's lane-group width L and pieces per lane NP for a head
// dim: the instantiated (L, NP) that covers it with the fewest idle piece
// slots (ties: the wider group).  D % 4 != 0 always takes L = 16.
struct GenPlan {
    int L, NP;
};
static GenPlan general_plan(int D, int extra) {
    // No 4-lane groups: measured at the config-5 shape they streamed at
    // 43-48% of HBM peak (D = 48, 80, 112), each load then touching 16
    // cache lines, against 70-79% for 8- and 16-lane groups.
    static const GenPlan vec4[] = {{16, 1}, {16, 2}, {16, 3}, {16, 4}, {16, 5}, {16, 6},
                                   {16, 8}, {16, 12}, {16, 16}, {8, 1}, {8, 2}, {8, 3},
                                   {8, 4}, {8, 5}, {8, 6}, {8, 7}};
    static const int np16[] = {1, 2, 3, 4, 5, 6, 8, 12, 16};
    if (D % 4 != 0) {
        const int need = (D + 63) / 64;
        for (int np : np16)
            if (np >= need) return {16, np};
        return {16, 16};
    }
    const int P = D / 4 + extra;
    GenPlan best{16, 16};
    int waste = 1 << 30;
    for (const GenPlan &g : vec4) {
        const int w = g.L * g.NP - P;
        if (w >= 0 && w < waste) {  // the table lists wider groups first
            waste = w;
            best = g;
        }
    }
    return best;
}

void paged_attention(const PagedArgs &a, hipStream_t s) {
    if (a.num_seqs <= 0 || a.num_heads <= 0) return;
    // Four heads per workgroup: measured at the benchmark shape, 2 heads
    // reached 79% and 8 heads 75-80% of HBM peak against 82% for 4.
    const dim3 grid((unsigned)((a.num_heads + 3) / 4), (unsigned)a.max_parts,
                    (unsigned)a.num_seqs);
    // CLOVE_PAGED_GENERAL=1 sends every shape to the general kernel (tests
    // and measurement of that kernel at the tuned shapes).
    const char *force = std::getenv("CLOVE_PAGED_GENERAL");
    const bool general = !paged_tuned(a.head_dim, a.block_size) || (force && *force == '1');
    if (general) {
        // Line-aligned pieces need room for the largest shift of any head:
        // 32 - gcd(D, 32) floats (D = 80 or 112: 16 floats, 4 pieces).
        PagedArgs ga = a;
        const int D = a.head_dim;
        int g32 = 32, d = D;
        while (d) {
            const int t = g32 % d;
            g32 = d;
            d = t;
        }
        const int extra = (32 - g32) / 4;
        ga.gen_shift = D % 4 == 0 && extra > 0 && ((int64_t)a.num_heads * D) % 32 == 0;
        const GenPlan g = general_plan(D, ga.gen_shift ? extra : 0);
        const int key = g.L * 100 + g.NP;
        // Head pairs (D = 16 or 48, H even): groups of 8 lanes, D / 16 pieces
        // (CLOVE_PAGED_PAIRS=0 turns them off, for tests and measurement).
        const char *pairs_env = std::getenv("CLOVE_PAGED_PAIRS");
        const bool head_pairs = (D == 16 || D == 48) && a.num_heads % 2 == 0 &&
                                !(pairs_env && *pairs_env == '0');
        if (head_pairs) {
            const dim3 grid2((unsigned)((a.num_heads / 2 + 3) / 4), (unsigned)a.max_parts,
                             (unsigned)a.num_seqs);
            if (D == 16) paged_general_kernel<8, 1, true, 2><<<grid2, 256, 0, s>>>(ga);
            else paged_general_kernel<8, 3, true, 2><<<grid2, 256, 0, s>>>(ga);
        } else if (a.head_dim % 4 != 0) {
            switch (key) {
#define CLOVE_PAGED_GEN1(L, NP)                                                    \
    case L * 100 + NP: paged_general_kernel<L, NP, false><<<grid, 256, 0, s>>>(ga); break;
                CLOVE_PAGED_GEN1(16, 1) CLOVE_PAGED_GEN1(16, 2) CLOVE_PAGED_GEN1(16, 3)
                CLOVE_PAGED_GEN1(16, 4) CLOVE_PAGED_GEN1(16, 5) CLOVE_PAGED_GEN1(16, 6)
                CLOVE_PAGED_GEN1(16, 8) CLOVE_PAGED_GEN1(16, 12) CLOVE_PAGED_GEN1(16, 16)
#undef CLOVE_PAGED_GEN1
                default: return;
            }
        } else {
            switch (key) {
#define CLOVE_PAGED_GEN4(L, NP)                                                    \
    case L * 100 + NP: paged_general_kernel<L, NP, true><<<grid, 256, 0, s>>>(ga); break;
                CLOVE_PAGED_GEN4(16, 1) CLOVE_PAGED_GEN4(16, 2) CLOVE_PAGED_GEN4(16, 3)
                CLOVE_PAGED_GEN4(16, 4) CLOVE_PAGED_GEN4(16, 5) CLOVE_PAGED_GEN4(16, 6)
                CLOVE_PAGED_GEN4(16, 8) CLOVE_PAGED_GEN4(16, 12) CLOVE_PAGED_GEN4(16, 16)
                CLOVE_PAGED_GEN4(8, 1) CLOVE_PAGED_GEN4(8, 2) CLOVE_PAGED_GEN4(8, 3)
                CLOVE_PAGED_GEN4(8, 4) CLOVE_PAGED_GEN4(8, 5) CLOVE_PAGED_GEN4(8, 6)
                CLOVE_PAGED_GEN4(8, 7)
#undef CLOVE_PAGED_GEN4
                default: return;
            }
        }
    } else {
#define CLOVE_PAGED_CASE(D, BS)                                                     \
    if (a.head_dim == D && a.block_size == BS) {                                    \
        paged_heads_kernel<D, BS, 4><<<grid, 256, 0, s>>>(a);                       \
    } else
        CLOVE_PAGED_CASE(64, 8) CLOVE_PAGED_CASE(64, 16) CLOVE_PAGED_CASE(64, 32)
        CLOVE_PAGED_CASE(128, 8) CLOVE_PAGED_CASE(128, 16) CLOVE_PAGED_CASE(128, 32)
        CLOVE_PAGED_CASE(256, 8) CLOVE_PAGED_CASE(256, 16) CLOVE_PAGED_CASE(256, 32)
        { return; }
#undef CLOVE_PAGED_CASE
    }
    const int pairs = a.num_seqs * a.num_heads;
    if (a.max_parts > 1)
        paged_merge_kernel<<<(unsigned)((pairs + 3) / 4), 256, 0, s>>>(a);
}

void paged_append(float *k_cache, float *v_cache, const float *k_new, const float *v_new,
                  const int32_t *block_tables, const int32_t *context_lens, int num_seqs,
                  int max_blocks, int block_size, int64_t num_blocks, int row_floats,
                  int32_t *err_flag, hipStream_t s) {
    if (num_seqs <= 0) return;
    paged_append_kernel<<<(unsigned)num_seqs, 256, 0, s>>>(k_cache, v_cache, k_new, v_new,
                                                          block_tables, context_lens, max_blocks,
                                                          block_size, num_blocks, row_floats,
                                                          err_flag);
}

void paged_slots(const int32_t *block_tables, const int32_t *context_lens, int32_t *slots,
                 int num_seqs, int max_blocks, int block_size, int max_ctx, int32_t *err_flag,
                 hipStream_t s) {
    const int64_t total = (int64_t)num_seqs * max_ctx;
    if (total <= 0) return;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    paged_slots_kernel<<<(unsigned)blocks, 256, 0, s>>>(block_tables, context_lens, slots,
                                                        num_seqs, max_blocks, block_size, max_ctx,
                                                        err_flag);
}

void paged_index_from_f32(const float *bt_f, int32_t *bt_out, const float *cl_f,
                          const int32_t *cl_i, int32_t *cl_out, int num_seqs, int max_blocks,
                          int block_size, int32_t *err_flag, hipStream_t s) {
    const int64_t total =
        (bt_f ? (int64_t)num_seqs * max_blocks : 0) + (cl_f ? (int64_t)num_seqs : 0);
    if (total <= 0) return;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    paged_index_kernel<<<(unsigned)blocks, 256, 0, s>>>(bt_f, bt_out, cl_f, cl_i, cl_out,
                                                        num_seqs, max_blocks, block_size,
                                                        err_flag);
}

}  // namespace k
}  // namespace clove
