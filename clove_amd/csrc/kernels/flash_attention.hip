// flash_attention.hip -- attention prefill (FlashAttention) and RoPE on CDNA4.
//
// Reference: the fused FlashAttention step of the lazy path (pattern
// MatMul -> Softmax -> MatMul with RoPE / ScalarMul on q and k, lazy.rs:
// 1621-1690; kernel lazy.rs:4821-4909) and the rope op (backend.rs:
// 2797-2826).  The WGSL runs one thread per query row of a single head,
// always applies RoPE and a causal mask, uses (1 + x/8)^8 for exp and keeps
// the key tile in a 1024-float array (so head_dim > 32 overflows it).  Here:
// batched, multi-head, causal and RoPE as flags, an exact exp, any length.
//
// Head dim 128: one workgroup = 4 waves = 128 queries of one (batch, head);
// each wave owns 32 queries (head dim 64 runs attention16_kernel of
// attention16.h: 16-query waves on the 16x16x4 MFMA, the same scheme
// otherwise; every other head dim runs that kernel from
// attention_general.hip).  Key blocks of 32 are staged through LDS
// (double-buffered, one barrier per block).  RoPE is applied before the kernel, once per element
// (a rotation inside it would be repeated by every query block that stages
// the same keys).  The products run on
// v_mfma_f32_32x32x2_f32 in TRANSPOSED form:
//   S^T = K . Q^T   (A = K tile from LDS, B = the wave's Q^T in registers)
//   O^T += V^T . P^T (A = V^T from LDS, B = P^T straight from S^T's registers)
// so lane l always works for query l%32: its S^T accumulator holds that
// query's scores for 16 of the block's 32 keys (the other 16 sit in lane
// l^32), and its O^T accumulator holds that query's output for 16 of every
// 32 head dimensions.  The online-softmax statistics (running max and sum)
// and the rescale of O are therefore per-lane scalars: a row reduction is
// 15 in-register ops plus one shuffle with lane l^32, and P never goes
// through LDS.  The K-group split of the GEMM kernel is reused: a 16-byte
// read of K / Q gives lane half h the four d values 8g + 4h .. 8g + 4h + 3,
// consumed one per MFMA step.
//
// Work order: workgroup L takes query block nqb-1 - L/(B*H) of (batch, head)
// L % (B*H).  Under the causal mask a query block's cost grows with its
// index, so this starts the heaviest blocks of every head first (a
// longest-first list schedule: with 64 slots per XCD at S = 4096, H = 32 its
// makespan is the ideal 33 block-units, where walking one head after another
// took 49).  Workgroups are dealt to the 8 XCDs round-robin (L % 8), so when
// B*H is a multiple of 8 each XCD serves a fixed set of heads and their K
// and V stay in its L2.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "attention16.h"
#include "launch.hpp"
#include "wave.h"

namespace clove {
namespace k {

namespace {

typedef float f16v __attribute__((ext_vector_type(16)));

template <int D, bool CAUSAL>
__global__ void __launch_bounds__(256, 2) attention_kernel(AttnArgs a) {
    constexpr int kPK = D + 4;  // K tile pitch (16-byte reads by 32 rows: no conflicts)
    constexpr int kPV = D + 8;  // V tile pitch (rows r and r+4 land 32 banks apart)
    constexpr int kG = D / 8;   // K-groups of 8 dims
    constexpr int kJ = D / 32;  // 32-dim blocks of O^T
    constexpr int kVec = kBK * D / 4 / 256;  // 16-byte tile loads per thread (K and V each)
    static_assert(kVec >= 1, "tile smaller than the workgroup");
    __shared__ __attribute__((aligned(16))) float sK[2][kBK * kPK];
    __shared__ __attribute__((aligned(16))) float sV[2][kBK * kPV];

    // heaviest query blocks first, heads interleaved (see the file comment)
    const int L = blockIdx.x;
    const int BH = a.B * a.H;
    const int qb = a.nqb - 1 - L / BH;
    const int bh = L % BH;
    const int h = bh % a.H, b = bh / a.H;

    const int HD = a.H * D;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l32 = lane & 31, hh = lane >> 5;
    const int q0 = qb * kBQ;
    const int query = q0 + wave * 32 + l32;
    const bool q_ok = query < a.S;
    const float *qrow = a.q + ((size_t)b * a.S + (q_ok ? query : 0)) * HD + (size_t)h * D;

    // this wave's Q^T fragment: dims 8g + 4hh .. +3 of its query, times the
    // softmax scale.  Scaling here also makes the Q loads complete before the
    // key loop: first used inside it, they would make the compiler wait for
    // every outstanding load (the next tile's included) at each block.
    // With RoPE, q's pairs (dims 8g + 4hh + {0,1} and {2,3}, whole pairs in
    // this lane) are rotated here, with the arithmetic of the RoPE pass
    // (rope_rows_kernel), before the scale: the same values that pass would
    // have stored, without its read and write of q.
    const float2 *trow = a.rope_tab && q_ok
                             ? a.rope_tab + (size_t)(query + a.q_pos - a.tab_pos0) * (D / 2)
                             : nullptr;
    // Scores are kept in base-2 units: q carries scale * log2(e), so a
    // softmax weight is exp2(s - m) with no multiply per score.
    const float qscale = a.scale * 1.44269504088896341f;
    cl_f4 qf[kG];
#pragma unroll
    for (int g = 0; g < kG; ++g) {
        cl_f4 v = q_ok ? *reinterpret_cast<const cl_f4 *>(qrow + 8 * g + 4 * hh)
                       : (cl_f4){0.f, 0.f, 0.f, 0.f};
        if (trow) {
            const float2 t0 = trow[4 * g + 2 * hh], t1 = trow[4 * g + 2 * hh + 1];
            cl_f4 r;
            r.x = v.x * t0.x - v.y * t0.y;
            r.y = v.x * t0.y + v.y * t0.x;
            r.z = v.z * t1.x - v.w * t1.y;
            r.w = v.z * t1.y + v.w * t1.x;
            v = r;
        }
        qf[g] = v * qscale;
    }

    // keys [0, k_end) can be visible to some query of the workgroup
    int k_end = a.Sk;
    if (CAUSAL) {
        const int last = min(q0 + kBQ - 1, a.S - 1) + a.q_pos - a.k_pos;
        k_end = min(k_end, last + 1);
    }
    // the same bound for this wave's queries (whole blocks past it are skipped)
    int k_wave = a.Sk;
    if (CAUSAL) k_wave = min(k_wave, min(q0 + wave * 32 + 31, a.S - 1) + a.q_pos - a.k_pos + 1);
    const int nblk = k_end > 0 ? (k_end + kBK - 1) / kBK : 0;
    // this lane's query sees keys t < lim
    const int lim = q_ok ? (CAUSAL ? min(a.Sk, query + a.q_pos - a.k_pos + 1) : a.Sk) : 0;

    // K and V tiles come through buffer loads over this batch's [Sk, H*D]
    // rows: a key past Sk gets an offset past the end and reads as zeros.  A
    // guarded ordinary load would become a branch that the compiler closes
    // with a wait for all loads, which exposes the whole load latency of
    // every block instead of overlapping it with the block before.
    constexpr uint32_t kOutside = 0x80000000u;  // the host keeps Sk*H*D*4 < 2^31
    const uint32_t kv_bytes = (uint32_t)a.Sk * (uint32_t)HD * 4u;
    const __amdgpu_buffer_rsrc_t rsrc_k = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(a.k + (size_t)b * a.Sk * HD), (short)0, (int)kv_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsrc_v = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(a.v + (size_t)b * a.Sk * HD), (short)0, (int)kv_bytes, 0x00020000);
    cl_f4 rk[kVec], rv[kVec];
    // Each load's offset within the tile (key and dims) is fixed per lane;
    // the block's first key enters as the scalar offset, so a block of keys
    // all below Sk costs no per-lane arithmetic.  (kb < Sk always, and the
    // host keeps Sk * H * D * 4 < 2^31, so the scalar offset cannot carry
    // kOutside round.)
    uint32_t toff[kVec];
    int tkey[kVec];
#pragma unroll
    for (int i = 0; i < kVec; ++i) {
        const int idx = threadIdx.x + 256 * i;
        const int key = idx / (D / 4), dq = idx % (D / 4);
        tkey[i] = key;
        toff[i] = ((uint32_t)key * (uint32_t)HD + (uint32_t)(h * D + 4 * dq)) * 4u;
    }
    auto load_tile = [&](int kb) {
        const int soff = kb * HD * 4;
        uint32_t off[kVec];
#pragma unroll
        for (int i = 0; i < kVec; ++i) off[i] = toff[i];
        if (kb + kBK > a.Sk) {  // the last block: keys past Sk read as zeros
            asm volatile("");   // (keeps this a branch, not selects every block pays for)
#pragma unroll
            for (int i = 0; i < kVec; ++i) off[i] = kb + tkey[i] < a.Sk ? toff[i] : kOutside;
        }
#pragma unroll
        for (int i = 0; i < kVec; ++i) {
            rk[i] = __builtin_bit_cast(cl_f4, __builtin_amdgcn_raw_buffer_load_b128(rsrc_k, (int)off[i], soff, 0));
            rv[i] = __builtin_bit_cast(cl_f4, __builtin_amdgcn_raw_buffer_load_b128(rsrc_v, (int)off[i], soff, 0));
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < kVec; ++i) {
            const int idx = threadIdx.x + 256 * i;
            const int key = idx / (D / 4), dq = idx % (D / 4);
            *reinterpret_cast<cl_f4 *>(&sK[buf][key * kPK + 4 * dq]) = rk[i];
            *reinterpret_cast<cl_f4 *>(&sV[buf][key * kPV + 4 * dq]) = rv[i];
        }
    };

    float m = -INFINITY, lsum = 0.0f;
    f16v o[kJ];
#pragma unroll
    for (int j = 0; j < kJ; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[j][e] = 0.f;

    if (nblk > 0) {
        load_tile(0);
        store_tile(0);
    }
    __syncthreads();
    for (int blk = 0; blk < nblk; ++blk) {
        const int kb = blk * kBK;
        const int cur = blk & 1;
        const bool more = blk + 1 < nblk;
        if (more) load_tile(kb + kBK);

        if (kb < k_wave) {
            const float *K = sK[cur];
            const float *V = sV[cur];
            // S^T = K . Q^T: s[i] is the score of key kb + 8(i/4) + 4hh + i%4
            // (in base-2 units).  One accumulator: splitting the chain over
            // two measured the same and cost 16 adds per block.
            f16v s;
#pragma unroll
            for (int e = 0; e < 16; ++e) s[e] = 0.f;
            // Raised wave priority over the two MFMA blocks (QK and PV): a
            // wave issuing MFMAs keeps the arbiter while the other waves on
            // its SIMD do their softmax VALU work, tile loads and stores in
            // the gaps (S = 4096, H = 32, D = 128: 116.2 -> 124.9 TFLOP/s,
            // same results bit for bit).
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int g = 0; g < kG; ++g) {
                const cl_f4 kf = *reinterpret_cast<const cl_f4 *>(K + l32 * kPK + 8 * g + 4 * hh);
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[t], qf[g][t], s, 0, 0, 0);
            }
            __builtin_amdgcn_s_setprio(0);
            // A block the whole wave sees (every key < Sk and, under the causal
            // mask, at or before the wave's first query) skips the mask.
            // The empty asm statement keeps the mask a branch: without it the
            // compiler turns it into selects that every block pays for.
            const int qw0 = q0 + wave * 32;
            bool full = kb + kBK <= a.Sk && qw0 + 32 <= a.S;
            if (CAUSAL) full = full && kb + kBK - 1 + a.k_pos <= qw0 + a.q_pos;
            if (!full) {
                asm volatile("");
                const int vis = lim - kb - 4 * hh;  // s[i] visible iff 8(i/4) + i%4 < vis
#pragma unroll
                for (int i = 0; i < 16; ++i) s[i] = 8 * (i / 4) + (i % 4) < vis ? s[i] : -INFINITY;
            }
            float mloc = -INFINITY;
#pragma unroll
            for (int i = 0; i < 16; ++i) mloc = fmaxf(mloc, s[i]);
            mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
            // Lazy rescale: the running max m moves only when some query of the
            // wave sees a score more than kSlack above it.  Scores up to
            // m + kSlack give weights up to 2^kSlack, harmless in f32, and the
            // numerator O and the denominator lsum share m, so the result is
            // the same; the 16*kJ-multiply rescale of O is skipped on most
            // blocks.  (m = -inf, no visible key yet, always updates.)
            constexpr float kSlack = 8.0f;
            const bool grow = __any(mloc > m + kSlack);
            if (grow) {
                const float m_new = fmaxf(m, mloc);
                const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m - m_new);
                lsum *= alpha;
#pragma unroll
                for (int j = 0; j < kJ; ++j)
#pragma unroll
                    for (int e = 0; e < 16; ++e) o[j][e] *= alpha;
                m = m_new;
            }
            // exp2(-inf) is 0, so masked scores need no test; only a lane
            // with no visible key yet (m = -inf, every score of the block
            // -inf) takes 0 as its max so that -inf - m is not NaN.
            const float mz = m == -INFINITY ? 0.0f : m;
            float ps = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                s[i] = __builtin_amdgcn_exp2f(s[i] - mz);
                ps += s[i];
            }
            ps += __shfl_xor(ps, 32, 64);
            lsum += ps;
            // O^T += V^T . P^T (step i pairs key 8(i/4)+i%4 of half 0 with key
            // 8(i/4)+4+i%4 of half 1, as S^T's layout holds them)
            // the kJ output blocks are independent accumulators: consecutive
            // MFMAs alternate between them
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int key = 8 * (i / 4) + 4 * hh + (i % 4);
#pragma unroll
                for (int j = 0; j < kJ; ++j) {
                    const float vv = V[key * kPV + 32 * j + l32];
                    o[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv, s[i], o[j], 0, 0, 0);
                }
                // bound how far the V reads are hoisted (all 64 at once cost 64
                // registers and an occupancy step)
                if (i % 4 == 3) __builtin_amdgcn_sched_barrier(0);
            }
        }
        __builtin_amdgcn_s_setprio(0);
        if (more) store_tile(cur ^ 1);
        __syncthreads();
    }

    if (!q_ok) return;
    // o[j][e] = O[query][32j + 8(e/4) + 4hh + e%4]: four consecutive dims per e/4
    const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
    float *orow = a.out + ((size_t)b * a.S + query) * HD + (size_t)h * D;
#pragma unroll
    for (int j = 0; j < kJ; ++j)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const cl_f4 r = {o[j][4 * u] * inv, o[j][4 * u + 1] * inv, o[j][4 * u + 2] * inv,
                             o[j][4 * u + 3] * inv};
            *reinterpret_cast<cl_f4 *>(orow + 32 * j + 8 * u + 4 * hh) = r;
        }
}

// Head dim 64 runs attention16_kernel (attention16.h): 16-query waves on
// v_mfma_f32_16x16x4_f32, 8 waves = 128 queries per workgroup.  Half the
// accumulators and Q registers of the 32-query form (77 VGPRs at D = 64), so
// three workgroups share a CU: six waves per SIMD to cover one another's
// softmax and LDS waits.  Measured at B = 1, S = 4096, H = 32, causal +
// RoPE: 0.595-0.600 ms against 0.672-0.673 ms for attention_kernel<64>
// (results within 1e-6 relative of it; the sums run in another order).  At
// D = 128 (120 VGPRs, four waves per SIMD) it ran within 2% of
// attention_kernel<128> either way and is not used there.

// RoPE table: tab[p][j] = (cos, sin) of theta = (pos0 + p) / div[j], the
// angle of pair j (dims 2j, 2j+1) at position pos0 + p (backend.rs:2818).
// Built once per call, so each (position, pair) pays one sincosf however
// many heads and rows use it.
__global__ void __launch_bounds__(256) rope_table_kernel(float2 *__restrict__ tab, int pos0,
                                                         int npos, int pairs, AttnFreq f) {
#pragma clang fp contract(off)
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= npos * pairs) return;
    const int p = i / pairs, j = i % pairs;
    const float theta = (float)(pos0 + p) / f.div[j];
    float s, c;
    sincosf(theta, &s, &c);
    tab[i] = make_float2(c, s);
}

// backend.rs:2797-2826: x1' = x1 cos - x2 sin, x2' = x1 sin + x2 cos per pair
// of every whole head; dims past the last whole head are written as 0.
// One workgroup of kRopeThreads threads per row (grid-stride over rows): the
// row's position and its table row are computed once, each thread then
// rotates 16-byte vectors (two pairs), issuing up to kRopeVec vector loads
// before any arithmetic.  512 threads x 2 vectors (a 4096-float row in one
// pass) streamed faster than 256 x 4 with inputs the last-level cache does
// not hold.
constexpr int kRopeThreads = 512, kRopeVec = 2;
// HD4 (head_dim % 4 == 0): a vector's two pairs are table entries 2m and
// 2m + 1 of one row, adjacent and 16-byte aligned, fetched with one 16-byte
// load issued with the row's loads; the whole-head bound then covers both
// pairs of a vector alike.
template <bool HD4>
__global__ void __launch_bounds__(kRopeThreads) rope_rows_kernel(const float *__restrict__ x,
                                                                 float *__restrict__ out,
                                                                 uint64_t rows, int seq,
                                                                 int hidden, int head_dim,
                                                                 int pos_offset, const float2 *tab,
                                                                 int tab_pos0) {
#pragma clang fp contract(off)
    const int nv = hidden / 4;
    const int pairs = head_dim / 2;
    const int whole = (hidden / head_dim) * head_dim;
    for (uint64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const int p = (int)(r % (uint64_t)seq) + pos_offset - tab_pos0;
        const float2 *trow = tab + (size_t)p * pairs;
        const float *xr = x + r * (uint64_t)hidden;
        float *orow = out + r * (uint64_t)hidden;
        for (int v0 = threadIdx.x; v0 < nv; v0 += kRopeVec * kRopeThreads) {
            cl_f4 xv[kRopeVec], tv[kRopeVec];
#pragma unroll
            for (int u = 0; u < kRopeVec; ++u) {
                const int v = v0 + kRopeThreads * u;
                if (v < nv) {
                    xv[u] = __builtin_nontemporal_load(reinterpret_cast<const cl_f4 *>(xr) + v);
                    if (HD4 && 4 * v < whole)
                        tv[u] = *reinterpret_cast<const cl_f4 *>(trow + ((4 * v) % head_dim) / 2);
                }
            }
#pragma unroll
            for (int u = 0; u < kRopeVec; ++u) {
                const int v = v0 + kRopeThreads * u;
                if (v >= nv) continue;
                const int c0 = 4 * v;
                cl_f4 o = {0.f, 0.f, 0.f, 0.f};
                if (HD4) {
                    if (c0 < whole) {
                        o.x = xv[u].x * tv[u].x - xv[u].y * tv[u].y;
                        o.y = xv[u].x * tv[u].y + xv[u].y * tv[u].x;
                        o.z = xv[u].z * tv[u].z - xv[u].w * tv[u].w;
                        o.w = xv[u].z * tv[u].w + xv[u].w * tv[u].z;
                    }
                } else {
                    if (c0 < whole) {
                        const float2 t0 = trow[(c0 % head_dim) / 2];
                        o.x = xv[u].x * t0.x - xv[u].y * t0.y;
                        o.y = xv[u].x * t0.y + xv[u].y * t0.x;
                    }
                    if (c0 + 2 < whole) {
                        const float2 t1 = trow[((c0 + 2) % head_dim) / 2];
                        o.z = xv[u].z * t1.x - xv[u].w * t1.y;
                        o.w = xv[u].z * t1.y + xv[u].w * t1.x;
                    }
                }
                __builtin_nontemporal_store(o, reinterpret_cast<cl_f4 *>(orow) + v);
            }
        }
    }
}

// Pair-at-a-time form for rows whose vectors are not 16-byte aligned.
__global__ void __launch_bounds__(256) rope_pairs_kernel(const float *__restrict__ x,
                                                         float *__restrict__ out, uint64_t rows,
                                                         int seq, int hidden, int head_dim,
                                                         int pos_offset, const float2 *tab,
                                                         int tab_pos0) {
#pragma clang fp contract(off)
    const int pairs = head_dim / 2;
    const int whole = (hidden / head_dim) * head_dim;
    for (uint64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const int p = (int)(r % (uint64_t)seq) + pos_offset - tab_pos0;
        const float2 *trow = tab + (size_t)p * pairs;
        const uint64_t base = r * (uint64_t)hidden;
        for (int c0 = 2 * threadIdx.x; c0 < hidden; c0 += 2 * 256) {
            float o0 = 0.0f, o1 = 0.0f;
            if (c0 < whole) {
                const float2 t = trow[(c0 % head_dim) / 2];
                const float x1 = x[base + c0], x2 = x[base + c0 + 1];
                o0 = x1 * t.x - x2 * t.y;
                o1 = x1 * t.y + x2 * t.x;
            }
            out[base + c0] = o0;
            out[base + c0 + 1] = o1;
        }
    }
}

}  // namespace

bool attention_supported(int head_dim) { return head_dim >= 1 && head_dim <= kAttnMaxHeadDim; }

void attention_prefill(const float *q, const float *k, const float *v, float *out, int B, int S,
                       int Sk, int H, int D, int q_pos, int k_pos, bool causal, float scale,
                       const float *q_rope_tab, int tab_pos0, hipStream_t s) {
    if (B <= 0 || S <= 0 || H <= 0) return;
    AttnArgs a{q, k, v, out, B, S, Sk, H, q_pos, k_pos, scale, 0,
               reinterpret_cast<const float2 *>(q_rope_tab), tab_pos0, D};
    a.nqb = (S + kBQ - 1) / kBQ;
    const unsigned grid = (unsigned)(B * H * a.nqb);
    if (D == 64) {
        if (causal) attention16_kernel<64, true, false, true><<<grid, 512, 0, s>>>(a);
        else attention16_kernel<64, false, false, true><<<grid, 512, 0, s>>>(a);
    } else if (D == 128) {
        if (causal) attention_kernel<128, true><<<grid, 256, 0, s>>>(a);
        else attention_kernel<128, false><<<grid, 256, 0, s>>>(a);
    } else {
        attention_prefill_general(a, causal, grid, s);
    }
}

void rope_table(float *tab, int pos0, int npos, int head_dim, const AttnFreq &freq,
                hipStream_t s) {
    const int n = npos * (head_dim / 2);
    if (n <= 0) return;
    rope_table_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(
        reinterpret_cast<float2 *>(tab), pos0, npos, head_dim / 2, freq);
}

void rope_apply(const float *x, float *out, size_t rows, int seq, int hidden, int head_dim,
                int pos_offset, const float *tab, int tab_pos0, hipStream_t s) {
    if (rows == 0 || hidden <= 0) return;
    const bool vec = hidden % 4 == 0 &&
                     ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out)) & 15) == 0;
    // one workgroup per row, at most 64 per CU's worth of rows in flight
    const unsigned grid = (unsigned)(rows < 16384 ? rows : 16384);
    const float2 *t = reinterpret_cast<const float2 *>(tab);
    if (vec && head_dim % 4 == 0)
        rope_rows_kernel<true><<<grid, kRopeThreads, 0, s>>>(x, out, rows, seq, hidden, head_dim,
                                                             pos_offset, t, tab_pos0);
    else if (vec)
        rope_rows_kernel<false><<<grid, kRopeThreads, 0, s>>>(x, out, rows, seq, hidden, head_dim,
                                                              pos_offset, t, tab_pos0);
    else
        rope_pairs_kernel<<<grid, 256, 0, s>>>(x, out, rows, seq, hidden, head_dim, pos_offset, t,
                                               tab_pos0);
}

}  // namespace k
}  // namespace clove
