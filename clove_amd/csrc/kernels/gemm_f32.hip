// gemm_f32.hip -- C = A.B in f32 on CDNA4 matrix cores.
//
// Reference: rayon_matmul (backend.rs:266-287) on the CPU and the 16x16
// LDS-tiled WGSL kernel (backend.rs:302-343, lazy.rs:4630-4659) on the GPU,
// which computes one output per thread with two LDS reads per FMA.
//
// Here each wavefront owns a WM x WN sub-tile built from 32x32 blocks of
// v_mfma_f32_32x32x2_f32 (64 cycles per instruction, 4096 FLOP), so one A
// and one B register feed 4096 FLOP.  A workgroup of four waves owns a
// BM x BN tile of C.  K advances in slabs of BK staged through LDS with two
// buffers: while the waves multiply slab s out of one buffer, the global
// loads of slab s+1 are already in flight and land in the other buffer, so a
// single barrier per slab orders the two.
//
// Operand layout.  v_mfma_f32_32x32x2_f32 reads, in lane l, A[l%32][l/32]
// and B[l/32][l%32], and returns D[8*(i/4) + 4*(l/32) + i%4][l%32] in
// accumulator element i.  The sum over k is order-free, so a K-group of 8 is
// split as k = 8g + 4h + t: lane half h = l/32 supplies the four k values
// 4h..4h+3 of the group from ONE 16-byte LDS read of A (A is kept row-major
// in LDS), and MFMA step t (t = 0..3) consumes component t.  B is kept
// k-major in LDS and read one float per step.
//
// Shapes: the fast path needs 16-byte aligned rows (K % 4 == 0 and
// N % 4 == 0); everything else, and every tile that crosses the edge of C,
// uses bounds-checked loads that fill zeros.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "launch.hpp"

namespace clove {
namespace k {

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));

struct GemmArgs {
    const float *A, *B;
    float *C;
    float *ws;        // split-K partial tiles [splits][tiles][BM*BN]
    int M, N, K, tiles_n, k_per_split, splits;
    GemmEpilogue epi;
};

// Epilogue: C = act(acc + bias[(row*N + col) % bias_n]), each step rounded
// in f32 exactly as Clove's separate Add (backend.rs:1489) and ReLU
// (:1823) / GELU (:1924) passes round it.
__device__ __forceinline__ float epilogue(const GemmEpilogue &e, float v, int row, int col, int N) {
#pragma clang fp contract(off)
    if (e.bias_mode == GEMM_BIAS_COL) v = v + e.bias[col];
    else if (e.bias_mode == GEMM_BIAS_SCALAR) v = v + e.bias[0];
    else if (e.bias_mode == GEMM_BIAS_MOD) v = v + e.bias[((uint64_t)row * N + col) % e.bias_n];
    if (e.act == GEMM_ACT_RELU) {
        v = v > 0.0f ? v : 0.0f;
    } else if (e.act == GEMM_ACT_GELU) {
        const float k = 0x1.988452p-1f;  // (2/pi).sqrt() in f32, backend.rs:1924
        const float x3 = (v * v) * v;
        v = 0.5f * v * (1.0f + tanhf(k * (v + 0.044715f * x3)));
    }
    return v;
}

template <int BM, int BN, int BK, int WM, int WN>
struct GemmCfg {
    static constexpr int kThreads = 256;
    static constexpr int kWavesN = BN / WN;
    static constexpr int kWavesM = BM / WM;
    static_assert(kWavesM * kWavesN == 4, "four waves per workgroup");
    static constexpr int kBlocksM = WM / 32;
    static constexpr int kBlocksN = WN / 32;
    static constexpr int kPitchA = BK + 4;    // floats; 16-byte aligned, breaks bank aliasing
    static constexpr int kPitchB = BN + 4;
    static constexpr int kSizeA = BM * kPitchA;
    static constexpr int kSizeB = BK * kPitchB;
    static constexpr int kLoadsA = BM * BK / 4 / kThreads;  // 16-byte loads per thread
    static constexpr int kLoadsB = BK * BN / 4 / kThreads;
    static_assert(kLoadsA >= 1 && kLoadsB >= 1, "tile too small for 256 threads");
    static_assert(BK % 8 == 0, "K slab is a whole number of 8-groups");
};

// Loads one slab of A (rows m0.., cols k0..) and B (rows k0.., cols n0..)
// into registers.  EDGE enables bounds checks; VEC selects 16-byte loads
// (only legal when K % 4 == 0 and N % 4 == 0).
template <class C, int BK, int BN, bool EDGE, bool VEC>
__device__ __forceinline__ void load_slab(const float *__restrict__ A, const float *__restrict__ B,
                                          int M, int N, int K, int m0, int n0, int k0, f4 *ra,
                                          f4 *rb) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < C::kLoadsA; ++i) {
        const int idx = tid + i * C::kThreads;
        const int r = idx / (BK / 4), kq = idx % (BK / 4);
        const int gm = m0 + r, gk = k0 + 4 * kq;
        const float *p = A + (size_t)gm * K + gk;
        if (!EDGE) {
            ra[i] = *reinterpret_cast<const f4 *>(p);
        } else if (VEC) {
            ra[i] = (gm < M && gk < K) ? *reinterpret_cast<const f4 *>(p) : (f4){0.f, 0.f, 0.f, 0.f};
        } else {
            f4 v;
            v.x = (gm < M && gk + 0 < K) ? p[0] : 0.f;
            v.y = (gm < M && gk + 1 < K) ? p[1] : 0.f;
            v.z = (gm < M && gk + 2 < K) ? p[2] : 0.f;
            v.w = (gm < M && gk + 3 < K) ? p[3] : 0.f;
            ra[i] = v;
        }
    }
#pragma unroll
    for (int i = 0; i < C::kLoadsB; ++i) {
        const int idx = tid + i * C::kThreads;
        const int r = idx / (BN / 4), nq = idx % (BN / 4);
        const int gk = k0 + r, gn = n0 + 4 * nq;
        const float *p = B + (size_t)gk * N + gn;
        if (!EDGE) {
            rb[i] = *reinterpret_cast<const f4 *>(p);
        } else if (VEC) {
            rb[i] = (gk < K && gn < N) ? *reinterpret_cast<const f4 *>(p) : (f4){0.f, 0.f, 0.f, 0.f};
        } else {
            f4 v;
            v.x = (gk < K && gn + 0 < N) ? p[0] : 0.f;
            v.y = (gk < K && gn + 1 < N) ? p[1] : 0.f;
            v.z = (gk < K && gn + 2 < N) ? p[2] : 0.f;
            v.w = (gk < K && gn + 3 < N) ? p[3] : 0.f;
            rb[i] = v;
        }
    }
}

template <class C, int BK, int BN>
__device__ __forceinline__ void store_slab(float *sA, float *sB, const f4 *ra, const f4 *rb) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < C::kLoadsA; ++i) {
        const int idx = tid + i * C::kThreads;
        const int r = idx / (BK / 4), kq = idx % (BK / 4);
        *reinterpret_cast<f4 *>(sA + r * C::kPitchA + 4 * kq) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < C::kLoadsB; ++i) {
        const int idx = tid + i * C::kThreads;
        const int r = idx / (BN / 4), nq = idx % (BN / 4);
        *reinterpret_cast<f4 *>(sB + r * C::kPitchB + 4 * nq) = rb[i];
    }
}

template <int BM, int BN, int BK, int WM, int WN, bool EDGE, bool VEC, bool EPI>
__global__ void __launch_bounds__(256) gemm_f32_mfma_kernel(GemmArgs g) {
    using Cfg = GemmCfg<BM, BN, BK, WM, WN>;
    __shared__ __attribute__((aligned(16))) float smem[2 * (Cfg::kSizeA + Cfg::kSizeB)];
    const float *__restrict__ A = g.A;
    const float *__restrict__ B = g.B;
    const int M = g.M, N = g.N, K = g.K;

    const int tile = blockIdx.x;
    const int split = blockIdx.y;
    const int m0 = (tile / g.tiles_n) * BM;
    const int n0 = (tile % g.tiles_n) * BN;
    const int k_begin = split * g.k_per_split;
    const int k_len = min(g.k_per_split, K - k_begin);

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm0 = (wave / Cfg::kWavesN) * WM;
    const int wn0 = (wave % Cfg::kWavesN) * WN;
    const int l32 = lane & 31;
    const int h = lane >> 5;

    f16v acc[Cfg::kBlocksM][Cfg::kBlocksN];
#pragma unroll
    for (int i = 0; i < Cfg::kBlocksM; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::kBlocksN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    f4 ra[Cfg::kLoadsA], rb[Cfg::kLoadsB];
    const int slabs = (k_len + BK - 1) / BK;

    load_slab<Cfg, BK, BN, EDGE, VEC>(A, B, M, N, K, m0, n0, k_begin, ra, rb);
    store_slab<Cfg, BK, BN>(smem, smem + Cfg::kSizeA, ra, rb);
    __syncthreads();

    for (int s = 0; s < slabs; ++s) {
        float *sA = smem + (s & 1) * (Cfg::kSizeA + Cfg::kSizeB);
        float *sB = sA + Cfg::kSizeA;
        const bool more = s + 1 < slabs;
        if (more)
            load_slab<Cfg, BK, BN, EDGE, VEC>(A, B, M, N, K, m0, n0, k_begin + (s + 1) * BK, ra, rb);

#pragma unroll
        for (int gk = 0; gk < BK / 8; ++gk) {
            f4 a[Cfg::kBlocksM];
            float b[Cfg::kBlocksN][4];
#pragma unroll
            for (int i = 0; i < Cfg::kBlocksM; ++i)
                a[i] = *reinterpret_cast<const f4 *>(sA + (wm0 + 32 * i + l32) * Cfg::kPitchA +
                                                     8 * gk + 4 * h);
#pragma unroll
            for (int j = 0; j < Cfg::kBlocksN; ++j)
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    b[j][t] = sB[(8 * gk + 4 * h + t) * Cfg::kPitchB + wn0 + 32 * j + l32];
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int i = 0; i < Cfg::kBlocksM; ++i)
#pragma unroll
                    for (int j = 0; j < Cfg::kBlocksN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][t], b[j][t],
                                                                         acc[i][j], 0, 0, 0);
        }

        if (more) {
            float *nA = smem + ((s + 1) & 1) * (Cfg::kSizeA + Cfg::kSizeB);
            store_slab<Cfg, BK, BN>(nA, nA + Cfg::kSizeA, ra, rb);
        }
        __syncthreads();
    }

    // Accumulator element e of block (i, j) is tile element (r, c) with
    // r = wm0 + 32*i + 8*(e/4) + 4*h + e%4 and c = wn0 + 32*j + l%32.
    if (g.splits == 1) {
#pragma unroll
        for (int i = 0; i < Cfg::kBlocksM; ++i)
#pragma unroll
            for (int j = 0; j < Cfg::kBlocksN; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int row = m0 + wm0 + 32 * i + 8 * (e / 4) + 4 * h + (e % 4);
                    const int col = n0 + wn0 + 32 * j + l32;
                    if (!EDGE || (row < M && col < N))
                        g.C[(size_t)row * N + col] =
                            EPI ? epilogue(g.epi, acc[i][j][e], row, col, N) : acc[i][j][e];
                }
        return;
    }

    // Split-K: park this split's tile; gemm_splitk_reduce sums the splits.
    float *part = g.ws + ((size_t)split * gridDim.x + tile) * (BM * BN);
#pragma unroll
    for (int i = 0; i < Cfg::kBlocksM; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::kBlocksN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int r = wm0 + 32 * i + 8 * (e / 4) + 4 * h + (e % 4);
                const int c = wn0 + 32 * j + l32;
                part[r * BN + c] = acc[i][j][e];
            }
}

// C[row][col] = sum over splits, in split order, of the parked tiles
// (deterministic).  One thread per four consecutive columns of a tile row.
__global__ void __launch_bounds__(256) gemm_splitk_reduce(const float *__restrict__ ws,
                                                          float *__restrict__ C, int M, int N,
                                                          int BM, int BN, int tiles_n, int tiles,
                                                          int splits, GemmEpilogue epi) {
    const int quads_per_row = BN / 4;
    const int64_t total = (int64_t)tiles * BM * quads_per_row;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * 256) {
        const int tile = (int)(i / ((int64_t)BM * quads_per_row));
        const int rem = (int)(i % ((int64_t)BM * quads_per_row));
        const int r = rem / quads_per_row, c = 4 * (rem % quads_per_row);
        const int row = (tile / tiles_n) * BM + r;
        const int col = (tile % tiles_n) * BN + c;
        if (row >= M || col >= N) continue;
        const size_t off = (size_t)tile * BM * BN + (size_t)r * BN + c;
        f4 sum = *reinterpret_cast<const f4 *>(ws + off);
        for (int sp = 1; sp < splits; ++sp)
            sum += *reinterpret_cast<const f4 *>(ws + (size_t)sp * tiles * BM * BN + off);
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (col + q < N) C[(size_t)row * N + col + q] = epilogue(epi, sum[q], row, col + q, N);
    }
}

// Tile configurations: (BM, BN, BK, WM, WN).
enum { CFG_32x128 = 0, CFG_64x64 = 1, CFG_128x128 = 2, CFG_128x128_K32 = 3, CFG_256x128 = 4,
       CFG_128x256 = 5, CFG_COUNT = 6 };
const int kCfgBM[CFG_COUNT] = {32, 64, 128, 128, 256, 128};
const int kCfgBN[CFG_COUNT] = {128, 64, 128, 128, 128, 256};
const int kCfgBK[CFG_COUNT] = {32, 16, 16, 32, 16, 16};

template <int BM, int BN, int BK, int WM, int WN>
void launch_cfg(const GemmPlan &p, GemmArgs g, hipStream_t s) {
    const dim3 grid((unsigned)p.tiles, (unsigned)p.splits);
    // The fused epilogue (bias modulo, GELU) costs registers; kernels without
    // one (and split-K kernels, whose reduce applies it) are built without it.
    const bool epi = p.splits == 1 &&
                     (g.epi.bias_mode != GEMM_BIAS_NONE || g.epi.act != GEMM_ACT_NONE);
    if (epi) {
        if (p.interior)
            gemm_f32_mfma_kernel<BM, BN, BK, WM, WN, false, true, true><<<grid, 256, 0, s>>>(g);
        else if (p.vec)
            gemm_f32_mfma_kernel<BM, BN, BK, WM, WN, true, true, true><<<grid, 256, 0, s>>>(g);
        else
            gemm_f32_mfma_kernel<BM, BN, BK, WM, WN, true, false, true><<<grid, 256, 0, s>>>(g);
    } else {
        if (p.interior)
            gemm_f32_mfma_kernel<BM, BN, BK, WM, WN, false, true, false><<<grid, 256, 0, s>>>(g);
        else if (p.vec)
            gemm_f32_mfma_kernel<BM, BN, BK, WM, WN, true, true, false><<<grid, 256, 0, s>>>(g);
        else
            gemm_f32_mfma_kernel<BM, BN, BK, WM, WN, true, false, false><<<grid, 256, 0, s>>>(g);
    }
}

}  // namespace

GemmPlan gemm_plan(int M, int N, int K, int num_cus, int force_cfg) {
    GemmPlan p{};
    p.M = M;
    p.N = N;
    p.K = K;
    // 128x256 tiles measured ~3% faster than 128x128 at 4096^3; they are used
    // whenever they alone still give every CU a tile.
    int cfg = M <= 32 ? CFG_32x128 : (M <= 64 ? CFG_64x64 : CFG_128x128);
    if (cfg == CFG_128x128 && ((M + 127) / 128) * ((N + 255) / 256) >= num_cus) cfg = CFG_128x256;
    if (force_cfg >= 0 && force_cfg < CFG_COUNT) cfg = force_cfg;
    p.cfg = cfg;
    const int BM = kCfgBM[cfg], BN = kCfgBN[cfg], BK = kCfgBK[cfg];
    p.tiles_n = (N + BN - 1) / BN;
    p.tiles = ((M + BM - 1) / BM) * p.tiles_n;
    // Split K when the tiles alone cannot fill the chip: aim for about two
    // workgroups per CU, each split covering at least four K slabs.
    const int slabs = (K + BK - 1) / BK;
    int splits = 1;
    if (p.tiles < num_cus) {
        splits = (2 * num_cus + p.tiles - 1) / p.tiles;
        const int max_splits = slabs / 4 > 1 ? slabs / 4 : 1;
        if (splits > max_splits) splits = max_splits;
        if (splits > 64) splits = 64;
    }
    int slabs_per = (slabs + splits - 1) / splits;
    p.k_per_split = slabs_per * BK;
    p.splits = (K + p.k_per_split - 1) / p.k_per_split;
    p.ws_floats = p.splits > 1 ? (size_t)p.splits * p.tiles * BM * BN : 0;
    p.vec = (K % 4 == 0) && (N % 4 == 0);
    p.interior = p.vec && (M % BM == 0) && (N % BN == 0) && (K % BK == 0) &&
                 (p.k_per_split % BK == 0);
    return p;
}

void gemm_f32(const GemmPlan &p, const float *A, const float *B, float *C, float *ws,
              const GemmEpilogue &epi, hipStream_t s) {
    if (p.M <= 0 || p.N <= 0) return;
    if (p.K <= 0) {
        (void)hipMemsetAsync(C, 0, (size_t)p.M * p.N * sizeof(float), s);
        return;
    }
    GemmPlan q = p;
    if (((reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B)) & 15) != 0) {
        q.vec = false;
        q.interior = false;
    }
    GemmArgs g{A, B, C, ws, p.M, p.N, p.K, p.tiles_n, p.k_per_split, p.splits, epi};
    switch (q.cfg) {
    case CFG_32x128: launch_cfg<32, 128, 32, 32, 32>(q, g, s); break;
    case CFG_64x64: launch_cfg<64, 64, 16, 32, 32>(q, g, s); break;
    case CFG_128x128: launch_cfg<128, 128, 16, 64, 64>(q, g, s); break;
    case CFG_128x128_K32: launch_cfg<128, 128, 32, 64, 64>(q, g, s); break;
    case CFG_256x128: launch_cfg<256, 128, 16, 128, 64>(q, g, s); break;
    default: launch_cfg<128, 256, 16, 64, 128>(q, g, s); break;
    }
    if (p.splits > 1) {
        const int BM = kCfgBM[q.cfg], BN = kCfgBN[q.cfg];
        const int64_t work = (int64_t)p.tiles * BM * (BN / 4);
        int64_t blocks = (work + 255) / 256;
        if (blocks > 8192) blocks = 8192;
        gemm_splitk_reduce<<<(unsigned)blocks, 256, 0, s>>>(ws, C, p.M, p.N, BM, BN, p.tiles_n,
                                                            p.tiles, p.splits, epi);
    }
}

}  // namespace k
}  // namespace clove
