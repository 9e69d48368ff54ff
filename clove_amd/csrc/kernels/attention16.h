// attention16.h -- the 16-query-per-wave attention prefill kernel on
// v_mfma_f32_16x16x4_f32, shared by flash_attention.hip (head dim 64, the
// fixed-shape build) and attention_general.hip (every other head dim).
//
// 8 waves = 128 queries per workgroup, the K and V tiles (32 or 64 keys,
// double buffered through LDS, one barrier per block) shared by all of them.
// Lane (r, q) = (l % 16, l / 16) works for query r of its wave:
//   S^T = K . Q^T per 16-key half hk, step (g, t) pairing K[hk*16 + r][16g +
//   4q + t] with Q[r][16g + 4q + t] (one 16-byte read of K per g);
//   element i of S^T half hk is key hk*16 + 4q + i of query r;
//   O^T += V^T . P^T, step (hk, i) pairing V[hk*16 + 4q + i][16jd + r] with
//   the lane's own P element i: no shuffles; element e of O^T block jd is
//   dim 16jd + 4q + e of query r.
//
// DP is the head dim the tiles are laid out for (a multiple of 16).  With
// GEN the real head dim D = a.D <= DP arrives at run time: dims at or past D
// load as zero in Q, K and V (zero terms in q . k; output dims that are never
// stored), so one instantiation serves every D in (DP - 16, DP].  VEC4 moves
// 16-byte pieces (D % 4 == 0, 16-byte aligned rows); without it every float
// moves on its own (any D, 4-byte alignment) and RoPE on q is applied by the
// caller beforehand.
//
// Work order: workgroup L takes query block nqb-1 - L/(B*H) of (batch, head)
// L % (B*H), so under the causal mask the heaviest blocks start first.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <type_traits>

#include "launch.hpp"
#include "wave.h"

namespace clove {
namespace k {

constexpr int kBQ = 128;  // queries per workgroup
constexpr int kBK = 32;   // keys per block

struct AttnArgs {
    const float *q, *k, *v;
    float *out;
    int B, S, Sk, H;
    int q_pos, k_pos;
    float scale;
    int nqb;                 // query blocks per (batch, head)
    const float2 *rope_tab;  // (cos, sin) per (position, pair) to rotate q, or null
    int tab_pos0;            // position of rope_tab's first row
    int D;                   // head dim (the GEN kernels read it; others use their DP)
};

template <int DP, bool CAUSAL, bool GEN, bool VEC4>
__global__ void __launch_bounds__(512, (DP <= 128 ? 4 : 2)) attention16_kernel(AttnArgs a) {
    static_assert(DP % 16 == 0, "tiles are laid out in 16-dim groups");
    static_assert(VEC4 || GEN, "the fixed-shape build moves 16-byte pieces");
    // pitches measured conflict-free at DP = 64 and 128 (SQ_LDS_BANK_CONFLICT 0):
    // a K read takes 16 rows x two 16-byte slots, a PV step 4 rows x 16 floats
    constexpr int kPK = DP + 8;
    constexpr int kPV = DP + 4;
    constexpr int kG = DP / 16;  // 16-dim groups of QK^T = 16-dim blocks of O^T
    // keys per block: 64 at DP = 16 and 64 (half the barriers per key; at
    // DP = 64 the 70 KiB of tiles still let two workgroups share a CU), 32
    // elsewhere.  S = 4096, H = 32, causal + RoPE, against 32: DP = 64
    // 0.578-0.631 against 0.604-0.667 ms (non-causal 1.034 against 1.067),
    // DP = 16 0.203 against 0.214 ms; DP = 32 and 48 lost 3-5%.
    constexpr int BK = (DP == 16 || DP == 64) ? 64 : kBK;
    constexpr int HK = BK / 16;  // 16-key halves of a block
    // tile elements (16-byte pieces, or floats) and per-thread loads, K and V each
    constexpr int kElems = VEC4 ? BK * DP / 4 : BK * DP;
    constexpr int kPer = (kElems + 511) / 512;
    constexpr int kRowElems = VEC4 ? DP / 4 : DP;
    using TileT = typename std::conditional<VEC4, cl_f4, float>::type;
    __shared__ __attribute__((aligned(16))) float sK[2][BK * kPK];
    __shared__ __attribute__((aligned(16))) float sV[2][BK * kPV];

    const int D = GEN ? a.D : DP;
    const int L = blockIdx.x;
    const int BH = a.B * a.H;
    const int qb = a.nqb - 1 - L / BH;
    const int bh = L % BH;
    const int h = bh % a.H, b = bh / a.H;

    const int HD = a.H * D;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, q4 = lane >> 4;
    const int q0 = qb * kBQ;
    const int qw0 = q0 + 16 * wave;
    const int query = qw0 + r16;
    const bool q_ok = query < a.S;
    const float *qrow = a.q + ((size_t)b * a.S + (q_ok ? query : 0)) * HD + (size_t)h * D;
    const float2 *trow = a.rope_tab && q_ok
                             ? a.rope_tab + (size_t)(query + a.q_pos - a.tab_pos0) * (D / 2)
                             : nullptr;
    // Scores are kept in base-2 units: q carries scale * log2(e), so a
    // softmax weight is exp2(s - m) with no multiply per score.
    const float qscale = a.scale * 1.44269504088896341f;
    cl_f4 qf[kG];
#pragma unroll
    for (int g = 0; g < kG; ++g) {
        const int d0 = 16 * g + 4 * q4;
        cl_f4 v = {0.f, 0.f, 0.f, 0.f};
        if (VEC4) {
            if (q_ok && (!GEN || d0 < D)) v = *reinterpret_cast<const cl_f4 *>(qrow + d0);
            // RoPE: q's pairs (dims d0 + {0,1} and {2,3}, whole pairs in this
            // lane) rotated with the arithmetic of the RoPE pass, before the
            // scale: the values that pass would have stored.
            if (trow && (!GEN || d0 < D)) {
                const float2 t0 = trow[d0 / 2], t1 = trow[d0 / 2 + 1];
                cl_f4 r;
                r.x = v.x * t0.x - v.y * t0.y;
                r.y = v.x * t0.y + v.y * t0.x;
                r.z = v.z * t1.x - v.w * t1.y;
                r.w = v.z * t1.y + v.w * t1.x;
                v = r;
            }
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (q_ok && d0 + e < D) v[e] = qrow[d0 + e];
        }
        qf[g] = v * qscale;
    }

    int k_end = a.Sk;
    if (CAUSAL) {
        const int last = min(q0 + kBQ - 1, a.S - 1) + a.q_pos - a.k_pos;
        k_end = min(k_end, last + 1);
    }
    int k_wave = a.Sk;
    if (CAUSAL) k_wave = min(k_wave, min(qw0 + 15, a.S - 1) + a.q_pos - a.k_pos + 1);
    const int nblk = k_end > 0 ? (k_end + BK - 1) / BK : 0;
    // this lane's query sees keys t < lim
    const int lim = q_ok ? (CAUSAL ? min(a.Sk, query + a.q_pos - a.k_pos + 1) : a.Sk) : 0;

    // K and V tiles come through buffer loads over this batch's [Sk, H*D]
    // rows: a key past Sk or a dim past D gets an offset past the end and
    // reads as zero.  A guarded ordinary load would become a branch that the
    // compiler closes with a wait for all loads, exposing each block's whole
    // load latency instead of overlapping it with the block before.
    constexpr uint32_t kOutside = 0x80000000u;  // the host keeps Sk*H*D*4 < 2^31
    const uint32_t kv_bytes = (uint32_t)a.Sk * (uint32_t)HD * 4u;
    const __amdgpu_buffer_rsrc_t rsrc_k = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(a.k + (size_t)b * a.Sk * HD), (short)0, (int)kv_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsrc_v = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(a.v + (size_t)b * a.Sk * HD), (short)0, (int)kv_bytes, 0x00020000);
    TileT rk[kPer], rv[kPer];
    // Each load's offset within the tile (key and dims, or kOutside for a
    // slot past the tile or a dim past D) is fixed per lane; the block's
    // first key enters as the scalar offset, so a block of keys all below Sk
    // costs no per-lane arithmetic.  (kb < Sk always, and the host keeps
    // Sk * H * D * 4 < 2^31, so the scalar offset cannot carry kOutside
    // round.)
    uint32_t toff[kPer];
    int tkey[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int idx = threadIdx.x + 512 * i;
        const int key = idx / kRowElems, dim = (idx % kRowElems) * (VEC4 ? 4 : 1);
        const bool ok = (kElems % 512 == 0 || idx < kElems) && (!GEN || dim < D);
        tkey[i] = key;
        toff[i] = ok ? ((uint32_t)key * (uint32_t)HD + (uint32_t)(h * D + dim)) * 4u : kOutside;
    }
    auto load_tile = [&](int kb) {
        const int soff = kb * HD * 4;
        uint32_t off[kPer];
#pragma unroll
        for (int i = 0; i < kPer; ++i) off[i] = toff[i];
        if (kb + BK > a.Sk) {  // the last block: keys past Sk read as zeros
            asm volatile("");   // (keeps this a branch, not selects every block pays for)
#pragma unroll
            for (int i = 0; i < kPer; ++i) off[i] = kb + tkey[i] < a.Sk ? toff[i] : kOutside;
        }
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            if constexpr (VEC4) {
                rk[i] = __builtin_bit_cast(TileT, __builtin_amdgcn_raw_buffer_load_b128(rsrc_k, (int)off[i], soff, 0));
                rv[i] = __builtin_bit_cast(TileT, __builtin_amdgcn_raw_buffer_load_b128(rsrc_v, (int)off[i], soff, 0));
            } else {
                rk[i] = __builtin_bit_cast(TileT, __builtin_amdgcn_raw_buffer_load_b32(rsrc_k, (int)off[i], soff, 0));
                rv[i] = __builtin_bit_cast(TileT, __builtin_amdgcn_raw_buffer_load_b32(rsrc_v, (int)off[i], soff, 0));
            }
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int idx = threadIdx.x + 512 * i;
            if (kElems % 512 != 0 && idx >= kElems) continue;
            const int key = idx / kRowElems, dim = (idx % kRowElems) * (VEC4 ? 4 : 1);
            *reinterpret_cast<TileT *>(&sK[buf][key * kPK + dim]) = rk[i];
            *reinterpret_cast<TileT *>(&sV[buf][key * kPV + dim]) = rv[i];
        }
    };

    float m = -INFINITY, lsum = 0.0f;
    cl_f4 o[kG];
#pragma unroll
    for (int j = 0; j < kG; ++j) o[j] = (cl_f4){0.f, 0.f, 0.f, 0.f};

    if (nblk > 0) {
        load_tile(0);
        store_tile(0);
    }
    __syncthreads();
    for (int blk = 0; blk < nblk; ++blk) {
        const int kb = blk * BK;
        const int cur = blk & 1;
        const bool more = blk + 1 < nblk;
        if (more) load_tile(kb + BK);

        if (kb < k_wave) {
            const float *K = sK[cur];
            const float *V = sV[cur];
            cl_f4 s[HK];
#pragma unroll
            for (int hk = 0; hk < HK; ++hk) s[hk] = (cl_f4){0.f, 0.f, 0.f, 0.f};
            // raised wave priority over the MFMA blocks: the other waves on
            // the SIMD do their softmax, tile loads and stores in the gaps
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int g = 0; g < kG; ++g)
#pragma unroll
                for (int hk = 0; hk < HK; ++hk) {
                    const cl_f4 kf =
                        *reinterpret_cast<const cl_f4 *>(K + (16 * hk + r16) * kPK + 16 * g + 4 * q4);
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        s[hk] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[t], qf[g][t], s[hk], 0, 0, 0);
                }
            __builtin_amdgcn_s_setprio(0);
            // A block the whole wave sees (every key < Sk and, under the causal
            // mask, at or before the wave's first query) skips the mask.
            // The empty asm statement keeps the mask a branch: without it the
            // compiler turns it into selects that every block pays for.
            bool full = kb + BK <= a.Sk && qw0 + 16 <= a.S;
            if (CAUSAL) full = full && kb + BK - 1 + a.k_pos <= qw0 + a.q_pos;
            if (!full) {
                asm volatile("");
                const int vis = lim - kb - 4 * q4;  // s[hk][i] visible iff 16hk + i < vis
#pragma unroll
                for (int hk = 0; hk < HK; ++hk)
#pragma unroll
                    for (int i = 0; i < 4; ++i) s[hk][i] = 16 * hk + i < vis ? s[hk][i] : -INFINITY;
            }
            float mloc = -INFINITY;
#pragma unroll
            for (int hk = 0; hk < HK; ++hk)
#pragma unroll
                for (int i = 0; i < 4; ++i) mloc = fmaxf(mloc, s[hk][i]);
            mloc = fmaxf(mloc, __shfl_xor(mloc, 16, 64));
            mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
            // Lazy rescale: the running max m moves only when some query of the
            // wave sees a score more than kSlack above it.  Scores up to
            // m + kSlack give weights up to 2^kSlack, harmless in f32, and the
            // numerator O and the denominator lsum share m, so the result is
            // the same; the rescale of O is skipped on most blocks.
            constexpr float kSlack = 8.0f;
            const bool grow = __any(mloc > m + kSlack);
            if (grow) {
                const float m_new = fmaxf(m, mloc);
                const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m - m_new);
                lsum *= alpha;
#pragma unroll
                for (int j = 0; j < kG; ++j) o[j] *= alpha;
                m = m_new;
            }
            // exp2(-inf) is 0, so masked scores need no test; only a lane
            // with no visible key yet takes 0 as its max so -inf - m is not NaN
            const float mz = m == -INFINITY ? 0.0f : m;
            float ps = 0.0f;
#pragma unroll
            for (int hk = 0; hk < HK; ++hk)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    s[hk][i] = __builtin_amdgcn_exp2f(s[hk][i] - mz);
                    ps += s[hk][i];
                }
            ps += __shfl_xor(ps, 16, 64);
            ps += __shfl_xor(ps, 32, 64);
            lsum += ps;
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int hk = 0; hk < HK; ++hk)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float *vr = V + (16 * hk + 4 * q4 + i) * kPV + r16;
#pragma unroll
                    for (int jd = 0; jd < kG; ++jd)
                        o[jd] = __builtin_amdgcn_mfma_f32_16x16x4f32(vr[16 * jd], s[hk][i], o[jd], 0, 0, 0);
                    __builtin_amdgcn_sched_barrier(0);
                }
        }
        __builtin_amdgcn_s_setprio(0);
        if (more) store_tile(cur ^ 1);
        __syncthreads();
    }

    if (!q_ok) return;
    const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
    float *orow = a.out + ((size_t)b * a.S + query) * HD + (size_t)h * D;
#pragma unroll
    for (int jd = 0; jd < kG; ++jd) {
        const int d0 = 16 * jd + 4 * q4;
        if (VEC4) {
            if (!GEN || d0 < D) *reinterpret_cast<cl_f4 *>(orow + d0) = o[jd] * inv;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (d0 + e < D) orow[d0 + e] = o[jd][e] * inv;
        }
    }
}

// Every head dim other than the fixed-shape builds' (attention_general.hip):
// a.D in [1, kAttnMaxHeadDim]; 16-byte rows when a.D % 4 == 0, else a
// null rope_tab (q already rotated).  grid = B * H * nqb workgroups.
void attention_prefill_general(const AttnArgs &a, bool causal, unsigned grid, hipStream_t s);

}  // namespace k
}  // namespace clove
