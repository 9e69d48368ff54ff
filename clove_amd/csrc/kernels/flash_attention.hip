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
// One workgroup = 4 waves = 128 queries of one (batch, head); each wave owns
// 32 queries.  Key blocks of 32 are staged through LDS (double-buffered, one
// barrier per block; K is rotated while it is staged).  The products run on
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
// Work order: the grid is walked so that all query blocks of one head land
// on the same XCD (blocks are dispatched round-robin over the 8 XCDs), so a
// head's K and V are fetched into one L2, and the heaviest (last, under the
// causal mask) query blocks start first.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "launch.hpp"
#include "wave.h"

namespace clove {
namespace k {

namespace {

typedef float f16v __attribute__((ext_vector_type(16)));

constexpr int kBQ = 128;  // queries per workgroup (4 waves x 32)
constexpr int kBK = 32;   // keys per block

struct AttnArgs {
    const float *q, *k, *v;
    float *out;
    int B, S, Sk, H;
    int q_pos, k_pos;
    float scale;
    int nqb;        // query blocks per (batch, head)
    int total;      // B * H * nqb
    int per_xcd;    // ceil(total / 8)
    AttnFreq freq;  // 10000^(2j/D), j < D/2, computed on the host with powf
};

__device__ __forceinline__ float fast_exp(float x) {
    return __builtin_amdgcn_exp2f(x * 1.44269504088896341f);
}

// Rotates the pairs (x, y) and (z, w) of f4 v holding dims d0..d0+3 at
// position pos (backend.rs:2819-2823: x1 cos - x2 sin, x1 sin + x2 cos).
__device__ __forceinline__ cl_f4 rope4(cl_f4 v, int d0, float pos, const AttnFreq &f) {
#pragma clang fp contract(off)
    const float t0 = pos / f.div[d0 / 2];
    const float t1 = pos / f.div[d0 / 2 + 1];
    float s0, c0, s1, c1;
    sincosf(t0, &s0, &c0);
    sincosf(t1, &s1, &c1);
    return (cl_f4){v.x * c0 - v.y * s0, v.x * s0 + v.y * c0, v.z * c1 - v.w * s1,
                   v.z * s1 + v.w * c1};
}

template <int D, bool CAUSAL, bool ROPE>
__global__ void __launch_bounds__(256) attention_kernel(AttnArgs a) {
    constexpr int kPK = D + 4;  // K tile pitch (16-byte reads by 32 rows: no conflicts)
    constexpr int kPV = D + 8;  // V tile pitch (rows r and r+4 land 32 banks apart)
    constexpr int kG = D / 8;   // K-groups of 8 dims
    constexpr int kJ = D / 32;  // 32-dim blocks of O^T
    constexpr int kVec = kBK * D / 4 / 256;  // 16-byte tile loads per thread (K and V each)
    static_assert(kVec >= 1, "tile smaller than the workgroup");
    __shared__ __attribute__((aligned(16))) float sK[2][kBK * kPK];
    __shared__ __attribute__((aligned(16))) float sV[2][kBK * kPV];

    // XCD-aware order: block L runs on XCD L % 8; consecutive work items
    // (the query blocks of one head) go to the same XCD.
    const int L = blockIdx.x;
    const int work = (L % 8) * a.per_xcd + L / 8;
    if (work >= a.total) return;
    const int qb = a.nqb - 1 - work % a.nqb;  // heaviest first
    const int bh = work / a.nqb;
    const int h = bh % a.H, b = bh / a.H;

    const int HD = a.H * D;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l32 = lane & 31, hh = lane >> 5;
    const int q0 = qb * kBQ;
    const int query = q0 + wave * 32 + l32;
    const bool q_ok = query < a.S;
    const float *qrow = a.q + ((size_t)b * a.S + (q_ok ? query : 0)) * HD + (size_t)h * D;

    // this wave's Q^T fragment: dims 8g + 4hh .. +3 of its query, rotated
    cl_f4 qf[kG];
#pragma unroll
    for (int g = 0; g < kG; ++g) {
        cl_f4 v = q_ok ? *reinterpret_cast<const cl_f4 *>(qrow + 8 * g + 4 * hh)
                       : (cl_f4){0.f, 0.f, 0.f, 0.f};
        if (ROPE) v = rope4(v, 8 * g + 4 * hh, (float)(query + a.q_pos), a.freq);
        qf[g] = v;
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

    const float *kbase = a.k + (size_t)b * a.Sk * HD + (size_t)h * D;
    const float *vbase = a.v + (size_t)b * a.Sk * HD + (size_t)h * D;
    cl_f4 rk[kVec], rv[kVec];
    auto load_tile = [&](int kb) {
#pragma unroll
        for (int i = 0; i < kVec; ++i) {
            const int idx = threadIdx.x + 256 * i;
            const int key = idx / (D / 4), dq = idx % (D / 4);
            const int t = kb + key;
            if (t < a.Sk) {
                rk[i] = *reinterpret_cast<const cl_f4 *>(kbase + (size_t)t * HD + 4 * dq);
                rv[i] = *reinterpret_cast<const cl_f4 *>(vbase + (size_t)t * HD + 4 * dq);
            } else {
                rk[i] = (cl_f4){0.f, 0.f, 0.f, 0.f};
                rv[i] = (cl_f4){0.f, 0.f, 0.f, 0.f};
            }
        }
    };
    auto store_tile = [&](int kb, int buf) {
#pragma unroll
        for (int i = 0; i < kVec; ++i) {
            const int idx = threadIdx.x + 256 * i;
            const int key = idx / (D / 4), dq = idx % (D / 4);
            cl_f4 kv = rk[i];
            if (ROPE) kv = rope4(kv, 4 * dq, (float)(kb + key + a.k_pos), a.freq);
            *reinterpret_cast<cl_f4 *>(&sK[buf][key * kPK + 4 * dq]) = kv;
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
        store_tile(0, 0);
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
            f16v s;
#pragma unroll
            for (int e = 0; e < 16; ++e) s[e] = 0.f;
#pragma unroll
            for (int g = 0; g < kG; ++g) {
                const cl_f4 kf = *reinterpret_cast<const cl_f4 *>(K + l32 * kPK + 8 * g + 4 * hh);
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[t], qf[g][t], s, 0, 0, 0);
            }
            float mloc = -INFINITY;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int t = kb + 8 * (i / 4) + 4 * hh + (i % 4);
                bool ok = t < a.Sk && q_ok;
                if (CAUSAL) ok = ok && t + a.k_pos <= query + a.q_pos;
                s[i] = ok ? s[i] * a.scale : -INFINITY;
                mloc = fmaxf(mloc, s[i]);
            }
            mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
            const float m_new = fmaxf(m, mloc);
            // m_new = -inf: no visible key yet for this query; keep zeros
            const float alpha = m_new == -INFINITY ? 1.0f : fast_exp(m - m_new);
            float ps = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                s[i] = s[i] == -INFINITY ? 0.0f : fast_exp(s[i] - m_new);
                ps += s[i];
            }
            ps += __shfl_xor(ps, 32, 64);
            lsum = lsum * alpha + ps;
            m = m_new;
            // O^T = alpha * O^T + V^T . P^T (step i pairs key 8(i/4)+i%4 of
            // half 0 with key 8(i/4)+4+i%4 of half 1, as S^T's layout holds them)
#pragma unroll
            for (int j = 0; j < kJ; ++j) {
#pragma unroll
                for (int e = 0; e < 16; ++e) o[j][e] *= alpha;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int key = 8 * (i / 4) + 4 * hh + (i % 4);
                    const float vv = V[key * kPV + 32 * j + l32];
                    o[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv, s[i], o[j], 0, 0, 0);
                }
            }
        }
        if (more) store_tile(kb + kBK, cur ^ 1);
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

// backend.rs:2797-2826: one thread per pair.
__global__ void __launch_bounds__(256) rope_kernel(const float *__restrict__ x,
                                                   float *__restrict__ out, uint64_t rows,
                                                   int seq, int hidden, int head_dim,
                                                   int pos_offset, AttnFreq f) {
#pragma clang fp contract(off)
    const int pairs_row = hidden / 2;
    const uint64_t total = rows * (uint64_t)pairs_row;
    for (uint64_t p = (uint64_t)blockIdx.x * 256 + threadIdx.x; p < total;
         p += (uint64_t)gridDim.x * 256) {
        const uint64_t r = p / pairs_row;
        const int c = 2 * (int)(p % pairs_row);
        const int head = c / head_dim, i = c % head_dim;
        const uint64_t idx = r * hidden + c;
        if ((head + 1) * head_dim > hidden) {  // past the last whole head: 0, as the
            out[idx] = 0.0f;                    // reference's zero-filled result leaves it
            out[idx + 1] = 0.0f;
            continue;
        }
        const float pos = (float)((int)(r % seq) + pos_offset);
        const float theta = pos / f.div[i / 2];
        float s, co;
        sincosf(theta, &s, &co);
        const float x1 = x[idx], x2 = x[idx + 1];
        out[idx] = x1 * co - x2 * s;
        out[idx + 1] = x1 * s + x2 * co;
    }
}

}  // namespace

bool attention_supported(int head_dim) { return head_dim == 64 || head_dim == 128; }

void attention_prefill(const float *q, const float *k, const float *v, float *out, int B, int S,
                       int Sk, int H, int D, int q_pos, int k_pos, int flags, float scale,
                       const AttnFreq &freq, hipStream_t s) {
    if (B <= 0 || S <= 0 || H <= 0) return;
    AttnArgs a{q, k, v, out, B, S, Sk, H, q_pos, k_pos, scale, 0, 0, 0, freq};
    a.nqb = (S + kBQ - 1) / kBQ;
    a.total = B * H * a.nqb;
    a.per_xcd = (a.total + 7) / 8;
    const unsigned grid = (unsigned)(a.per_xcd * 8);
    const bool causal = flags & ATTN_FLAG_CAUSAL, rope = flags & ATTN_FLAG_ROPE;
#define CLOVE_ATTN(DD)                                                                    \
    if (causal && rope) attention_kernel<DD, true, true><<<grid, 256, 0, s>>>(a);         \
    else if (causal) attention_kernel<DD, true, false><<<grid, 256, 0, s>>>(a);           \
    else if (rope) attention_kernel<DD, false, true><<<grid, 256, 0, s>>>(a);             \
    else attention_kernel<DD, false, false><<<grid, 256, 0, s>>>(a);
    if (D == 64) {
        CLOVE_ATTN(64)
    } else {
        CLOVE_ATTN(128)
    }
#undef CLOVE_ATTN
}

void rope(const float *x, float *out, size_t rows, int seq, int hidden, int head_dim,
          int pos_offset, const AttnFreq &freq, hipStream_t s) {
    const uint64_t total = rows * (uint64_t)(hidden / 2);
    if (!total) return;
    uint64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    rope_kernel<<<(unsigned)blocks, 256, 0, s>>>(x, out, rows, seq, hidden, head_dim, pos_offset,
                                                 freq);
}

}  // namespace k
}  // namespace clove
