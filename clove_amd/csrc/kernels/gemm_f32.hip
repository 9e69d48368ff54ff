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

#include <algorithm>

#include <cmath>
#include <cstdint>
#include <cstdlib>

#include "launch.hpp"

namespace clove {
namespace k {

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

// Raw buffer resource over [base, base + bytes): stride 0, word 3 = 32-bit
// data format (DATA_FORMAT = 4 in bits 15..18), the gfx9-family setting.
// Reads at offsets >= bytes return 0 (and a DMA lane past the end writes 0
// to LDS).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                             0x00020000);
}

struct GemmArgs {
    const float *A, *B;
    float *C;
    float *ws;        // split-K partial tiles [splits][tiles][BM*BN]
    int M, N, K, tiles_n, k_per_split, splits;
    GemmEpilogue epi;
    int tiles;        // tiles of C (the grid's x dimension is padded to 8 * per_xcd)
    int per_xcd;      // ceil(tiles / 8)
};

// Tile order.  Workgroups are dealt to the 8 XCDs round-robin (workgroup L
// runs on XCD L % 8), each with its own L2.  Workgroup L takes position
// V = (L % 8) * per_xcd + L / 8 of a grouped order, so each XCD walks one
// contiguous range of it; the grouped order visits kGroupM tile rows column
// by column.  At 4096^3 (32 x 16 tiles of 128 x 256) an XCD then owns an
// 8 x 8 block of tiles whose concurrently running workgroups share A and B
// slabs in its L2 (the plain row-major order gave each XCD 2 tile columns
// and all 32 tile rows, so every A slab was fetched for just two tiles).
constexpr int kGroupM = 8;
__device__ __forceinline__ bool gemm_tile(const GemmArgs &g, int *tile) {
    const int L = blockIdx.x;
    const int V = (L % 8) * g.per_xcd + L / 8;
    if (V >= g.tiles) return false;
    const int tiles_m = g.tiles / g.tiles_n;
    const int group_size = kGroupM * g.tiles_n;
    const int first = (V / group_size) * kGroupM;
    const int rows = min(kGroupM, tiles_m - first);
    const int r = V % group_size;
    *tile = (first + r % rows) * g.tiles_n + r / rows;
    return true;
}

// Epilogue: C = act(acc + bias[(row*N + col) % bias_n]), each step rounded
// in f32 exactly as Clove's separate Add (backend.rs:1489) and ReLU
// (:1823) / GELU (:1924) passes round it.
// bcol: bias[col] when the caller has loaded it already (GEMM_BIAS_COL), so
// that the load is not repeated after every store to C, which may alias it.
__device__ __forceinline__ float epilogue(const GemmEpilogue &e, float v, int row, int col, int N,
                                          const float *bcol = nullptr) {
#pragma clang fp contract(off)
    if (e.bias_mode == GEMM_BIAS_COL) v = v + (bcol ? *bcol : e.bias[col]);
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

// One accumulator element read out of its AGPR for the fused epilogue.
// Without it the compiler copies every accumulator of the wave into VGPRs
// when the K loop ends (128 more VGPRs at 128 x 256 and 256 x 128: one wave
// per SIMD instead of two, 4096^3 with bias + ReLU 1.128 ms against 0.973
// plain); read one at a time, the epilogue needs a few registers.
__device__ __forceinline__ float acc_read(float x) {
    float v;
    asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(x));
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

// Transposed-B slab: thread index idx moves k-quad kq of column n.  Lanes
// 16q .. 16q+15 of a wave take quad q of 16 consecutive columns, so one
// wave instruction reads 64 whole bytes of each of 16 rows of the [N, K]
// matrix, and the column stores of the four k values (rows 4kq + c of the
// B stage, pitch BN + 4) have no bank conflicts; four lanes per column (the
// quads of one row side by side) cost 2 conflict cycles per store
// (measured with SQ_LDS_BANK_CONFLICT on gfx950).
template <int BK>
__device__ __forceinline__ void tb_map(int idx, int *kq, int *n) {
    constexpr int KQ = BK / 4;
    *kq = (idx / 16) % KQ;
    *n = idx % 16 + 16 * (idx / (16 * KQ));
}

// Loads one slab of A (rows m0.., cols k0..) and B (rows k0.., cols n0..)
// into registers.  EDGE enables bounds checks; VEC selects 16-byte loads
// (only legal when K % 4 == 0 and N % 4 == 0).
// TA / TB (interior tiles only): A holds the [K, M] matrix whose transpose
// is the product's A, or B the [N, K] matrix whose transpose is its B.  A
// thread then loads four consecutive m (or k) of one k (or n) row, with k
// (or the k quad) the fastest index over the threads, and store_slab writes
// the four values to the same LDS places the plain layout would use, so the
// product is the same bit for bit as transposing first.
template <class C, int BM, int BK, int BN, bool EDGE, bool VEC, bool TA, bool TB>
__device__ __forceinline__ void load_slab(const float *__restrict__ A, const float *__restrict__ B,
                                          int M, int N, int K, int m0, int n0, int k0, f4 *ra,
                                          f4 *rb) {
    const int tid = threadIdx.x;
    static_assert(!(TA || TB) || (!EDGE && VEC), "transposed loads are interior-only");
    if constexpr (TA) {
#pragma unroll
        for (int i = 0; i < C::kLoadsA; ++i) {
            const int idx = tid + i * C::kThreads;
            const int k = idx % BK, mq = idx / BK;
            ra[i] = *reinterpret_cast<const f4 *>(A + (size_t)(k0 + k) * M + m0 + 4 * mq);
        }
    }
#pragma unroll
    for (int i = 0; i < (TA ? 0 : C::kLoadsA); ++i) {
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
    if constexpr (TB) {
#pragma unroll
        for (int i = 0; i < C::kLoadsB; ++i) {
            int kq, n;
            tb_map<BK>(tid + i * C::kThreads, &kq, &n);
            rb[i] = *reinterpret_cast<const f4 *>(B + (size_t)(n0 + n) * K + k0 + 4 * kq);
        }
    }
#pragma unroll
    for (int i = 0; i < (TB ? 0 : C::kLoadsB); ++i) {
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

// Float index of k-quad kq of row r in an A stage.  At BK = 16 the rows are
// unpadded and the quads of row r are XOR-permuted by (r >> 2) & 3: the
// MFMA operand reads (one ds_read_b128 per lane, rows l%32, quad 2g + l/32)
// then have no bank conflicts, where the padded pitch BK + 4 costs 12
// conflict cycles per read and the permutation by (r >> 1) & 3 costs 4
// (measured with SQ_LDS_BANK_CONFLICT on gfx950).  The transposed-A slab
// keeps the padded pitch: its stores write one column of rows 4 apart, and
// those rows must fall in different banks.
template <class C, int BK, bool TA>
__device__ __forceinline__ int a_pos(int r, int kq) {
    if constexpr (BK == 16 && !TA) return r * BK + 4 * (kq ^ ((r >> 2) & 3));
    else return r * C::kPitchA + 4 * kq;
}

template <class C, int BK, int BN, bool TA = false, bool TB = false>
__device__ __forceinline__ void store_slab(float *sA, float *sB, const f4 *ra, const f4 *rb) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < C::kLoadsA; ++i) {
        const int idx = tid + i * C::kThreads;
        if constexpr (TA) {  // four m of one k: column k of rows 4mq .. 4mq+3
            const int k = idx % BK, mq = idx / BK;
#pragma unroll
            for (int c = 0; c < 4; ++c) sA[(4 * mq + c) * C::kPitchA + k] = ra[i][c];
        } else {
            const int r = idx / (BK / 4), kq = idx % (BK / 4);
            *reinterpret_cast<f4 *>(sA + a_pos<C, BK, TA>(r, kq)) = ra[i];
        }
    }
#pragma unroll
    for (int i = 0; i < C::kLoadsB; ++i) {
        const int idx = tid + i * C::kThreads;
        if constexpr (TB) {  // four k of one n: rows 4kq .. 4kq+3 of column n
            int kq, n;
            tb_map<BK>(idx, &kq, &n);
#pragma unroll
            for (int c = 0; c < 4; ++c) sB[(4 * kq + c) * C::kPitchB + n] = rb[i][c];
        } else {
            const int r = idx / (BN / 4), nq = idx % (BN / 4);
            *reinterpret_cast<f4 *>(sB + r * C::kPitchB + 4 * nq) = rb[i];
        }
    }
}

template <int BM, int BN, int BK, int WM, int WN, bool EDGE, bool VEC, bool EPI, bool TA = false,
          bool TB = false>
__global__ void __launch_bounds__(256) gemm_f32_mfma_kernel(GemmArgs g) {
    using Cfg = GemmCfg<BM, BN, BK, WM, WN>;
    __shared__ __attribute__((aligned(16))) float smem[2 * (Cfg::kSizeA + Cfg::kSizeB)];
    const float *__restrict__ A = g.A;
    const float *__restrict__ B = g.B;
    const int M = g.M, N = g.N, K = g.K;

    int tile;
    if (!gemm_tile(g, &tile)) return;  // padding of the grid (before any barrier)
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

    load_slab<Cfg, BM, BK, BN, EDGE, VEC, TA, TB>(A, B, M, N, K, m0, n0, k_begin, ra, rb);
    store_slab<Cfg, BK, BN, TA, TB>(smem, smem + Cfg::kSizeA, ra, rb);
    __syncthreads();

    for (int s = 0; s < slabs; ++s) {
        float *sA = smem + (s & 1) * (Cfg::kSizeA + Cfg::kSizeB);
        float *sB = sA + Cfg::kSizeA;
        const bool more = s + 1 < slabs;
        if (more)
            load_slab<Cfg, BM, BK, BN, EDGE, VEC, TA, TB>(A, B, M, N, K, m0, n0,
                                                          k_begin + (s + 1) * BK, ra, rb);

        // Raised wave priority over the MFMA block: of the two workgroups
        // sharing a CU, the one issuing MFMAs keeps the arbiter, and the other
        // one's slab loads, stores and barrier wait slot into its gaps
        // (4096^3: 132.0 -> 137.6 TFLOP/s, same results bit for bit).
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int gk = 0; gk < BK / 8; ++gk) {
            f4 a[Cfg::kBlocksM];
            float b[Cfg::kBlocksN][4];
#pragma unroll
            for (int i = 0; i < Cfg::kBlocksM; ++i)
                a[i] = *reinterpret_cast<const f4 *>(
                    sA + a_pos<Cfg, BK, TA>(wm0 + 32 * i + l32, 2 * gk + h));
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
        __builtin_amdgcn_s_setprio(0);

        if (more) {
            float *nA = smem + ((s + 1) & 1) * (Cfg::kSizeA + Cfg::kSizeB);
            store_slab<Cfg, BK, BN, TA, TB>(nA, nA + Cfg::kSizeA, ra, rb);
        }
        __syncthreads();
    }

    // Accumulator element e of block (i, j) is tile element (r, c) with
    // r = wm0 + 32*i + 8*(e/4) + 4*h + e%4 and c = wn0 + 32*j + l%32.
    if (g.splits == 1) {
        float bc[Cfg::kBlocksN];  // per-column bias, loaded before any store
#pragma unroll
        for (int j = 0; j < Cfg::kBlocksN; ++j) {
            const int col = n0 + wn0 + 32 * j + l32;
            bc[j] = EPI && g.epi.bias_mode == GEMM_BIAS_COL && col < N ? g.epi.bias[col] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < Cfg::kBlocksM; ++i)
#pragma unroll
            for (int j = 0; j < Cfg::kBlocksN; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int row = m0 + wm0 + 32 * i + 8 * (e / 4) + 4 * h + (e % 4);
                    const int col = n0 + wn0 + 32 * j + l32;
                    // the epilogue is evaluated for every element (bc is 0
                    // past N, the modulo bias index is always in range): an
                    // accumulator read inside the bounds test stops the loop
                    // from unrolling, and the accumulators go to scratch
                    if constexpr (EPI) {
                        const float v =
                            epilogue(g.epi, acc_read(acc[i][j][e]), row, col, N, &bc[j]);
                        if (!EDGE || (row < M && col < N)) g.C[(size_t)row * N + col] = v;
                    } else {
                        if (!EDGE || (row < M && col < N)) g.C[(size_t)row * N + col] = acc[i][j][e];
                    }
                }
        return;
    }

    // Split-K: park this split's tile; gemm_splitk_reduce sums the splits.
    float *part = g.ws + ((size_t)split * g.tiles + tile) * (BM * BN);
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

// The 128 x 128, 128 x 256 and 64 x 128 configurations (tiles past M or N
// too: EDGE below), A and B under 2 GiB: the register-staged kernel's tile, waves and
// MFMA order with the slabs moved by buffer->LDS DMA instead of through
// registers.
// Each lane's 16 bytes land at its instruction's LDS base + 16 * lane, and
// the lane chooses which global 16 bytes it moves, so the LDS layout is set
// by the lane-to-address map:
//  * A stage [BM][BK]: 16-byte slot s of row r holds k-quad
//    s ^ ((r >> 2) & (BK/4 - 1)), the layout a_pos gives the register-staged
//    kernel (bank-conflict free at BK = 16, measured);
//  * B stage [BK][BN] at pitch BN (rows of 1 KiB at BN = 256): a lane's four
//    column blocks sit 32 floats apart in one row and pair up in ds_read2_b32.
//  * TA (the product's A is the transpose of the [K, M] matrix given): the
//    A stage is k-major [BK][BM], each lane moving four m of one k, and a
//    wave reads one float per MFMA step as it reads B;
//  * TB (B is the transpose of the [N, K] matrix given): the B stage is
//    n-major [BN][BK] with A's XOR layout, each lane moving four k of one n,
//    so a lane's four k of one column come in one ds_read_b128.
//    Both read the same values into the same MFMA steps as the plain
//    layouts, so the product is the same bit for bit as transposing first.
// ST slabs rotate through LDS (dma_stages below: three at 128 x 256, 72 KiB,
// two workgroups per CU; two at 128 x 128, 32 KiB, five workgroups per CU).
// Each wave waits for its own DMAs of slab s
// (vmcnt), then a bare s_barrier publishes them to the other waves:
// __syncthreads() carries a fence that would wait for every DMA in flight,
// the next slab's too.  A stage is refilled only after the barrier that
// follows its last reads (their values fed MFMAs issued before it).
// Measured at 4096^3 in 128 x 256 tiles on one box: 972 us (141 TFLOP/s)
// against 1005-1026 us for the register-staged form; double buffering (969
// us) and 256 x 256 tiles with 8 waves (961-982 us) within noise of it.
// Deeper slabs with one workgroup per CU (BK = 32 with 3 or 2 stages, BK =
// 16 with 4: 96-144 KiB of LDS) ran 1.020-1.047 ms against 0.963-0.967 ms,
// the same bits, and BK = 32 at 128 x 128 (two workgroups per CU) lost 3%:
// the other workgroups on a CU are what fill each one's barrier and LDS
// waits.
constexpr int kDmaStages = 3;
// 128 x 128 tiles keep two stages (32 KiB of LDS): four or five workgroups
// share a CU and hide each other's waits, where three stages (48 KiB) fit
// three.  Measured: 4096^3 in 128 x 128 tiles 0.973 against 1.201 ms, 5000
// x 4096 x 4096 1.228 against 1.484 ms.  128 x 256 tiles keep three (two
// stages ran 8192 x 4096 x 4096 at 2.384 against 1.939 ms).
constexpr int dma_stages(int BN) { return BN == 128 ? 2 : kDmaStages; }

// s_waitcnt immediate that waits until at most n vector-memory operations
// are outstanding (gfx9 encoding: vmcnt in bits 3:0 and 15:14; lgkmcnt and
// expcnt left at their maxima, so they are not waited for).
constexpr int vmcnt_imm(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }

// s_waitcnt until at most n vector-memory operations are outstanding, for an
// n that is a constant once the caller's loops are unrolled (rounded down to
// a multiple of 4 -- waiting for more is always safe -- and capped at 60).
__device__ __forceinline__ void wait_vmem(int n) {
    switch (n < 60 ? n / 4 : 15) {
#define CLOVE_WAIT_VMEM(i) \
    case i: __builtin_amdgcn_s_waitcnt(vmcnt_imm(4 * i)); break;
        CLOVE_WAIT_VMEM(0) CLOVE_WAIT_VMEM(1) CLOVE_WAIT_VMEM(2) CLOVE_WAIT_VMEM(3)
        CLOVE_WAIT_VMEM(4) CLOVE_WAIT_VMEM(5) CLOVE_WAIT_VMEM(6) CLOVE_WAIT_VMEM(7)
        CLOVE_WAIT_VMEM(8) CLOVE_WAIT_VMEM(9) CLOVE_WAIT_VMEM(10) CLOVE_WAIT_VMEM(11)
        CLOVE_WAIT_VMEM(12) CLOVE_WAIT_VMEM(13) CLOVE_WAIT_VMEM(14) CLOVE_WAIT_VMEM(15)
#undef CLOVE_WAIT_VMEM
        default: __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    }
}

// EDGE: tiles may reach past M or N, and K may end inside the last slab of
// the last split.  Rows of A past M and columns of B past N (N % 4 == 0, so
// a 16-byte piece is all in or all out) get the offset kOutside, past the
// end of both buffers, so the DMA writes zeros there whether or not the
// range check counts the slab step in soffset; kOutside plus any step
// (under K * N * 4 < 2^31) stays below 2^32.  In a last slab that K ends
// inside (K % 4 == 0: again whole pieces), A's pieces and B's rows past K
// get kOutside too, with the slab step moved into the unmasked offsets.
// A transposed operand takes the same masks: TA's pieces of four m past M
// (M % 4 == 0) and its rows past K, TB's rows past N and its pieces of four
// k past K (K % 4 == 0).  Stores and bias loads are bounds-checked.  The
// stored results are the same bits as the register-staged kernel's (and, for
// TA and TB, as transposing first), which also reads zeros there.
//
// Workgroups of the DMA kernel that fit one CU (one wave each per SIMD): the
// LDS ring's share of 160 KiB, and 512 registers a lane over the
// accumulators plus 40 more (four at 128 x 128).  Asking for five there
// (accumulators plus 32) made the fused-epilogue variants spill (their
// accumulators sit in AGPRs and a tighter budget is split between the two
// files) and the edge kernel slower: 5000 x 4096 x 4096 1.361 against 1.230
// ms, five co-resident workgroups against four and then one.
constexpr int dma_waves(int BM, int BN, int BK, int WM, int WN, int ST) {
    const int lds = (160 * 1024) / (ST * (BM * BK + BK * BN) * 4);
    const int regs = 512 / (((WM / 32) * (WN / 32) * 16 + 40 + 7) / 8 * 8);
    return lds < regs ? lds : regs;
}

// One buffer->LDS DMA of ONE float (4 bytes) or four (16 bytes) a lane.
template <bool ONE>
__device__ __forceinline__ void dma_lds(__amdgpu_buffer_rsrc_t r, float *dst, uint32_t voff,
                                        int soff) {
    if constexpr (ONE)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)dst, 4, (int)voff, soff, 0, 0);
    else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)dst, 16, (int)voff, soff, 0, 0);
}

// A1 / B1 (EDGE only): A's rows (K % 4 != 0) or B's rows (N % 4 != 0) are not
// 16-byte aligned, so that operand moves one float a lane (4-byte DMA) into
// the same LDS places, with the masks per element: the same bits again.
template <int BM, int BN, int BK, int WM, int WN, bool EPI, bool TA = false, bool TB = false,
          int ST = kDmaStages, bool EDGE = false, bool A1 = false, bool B1 = false>
__global__ void __launch_bounds__(256)
    __attribute__((amdgpu_waves_per_eu(dma_waves(BM, BN, BK, WM, WN, ST))))
    gemm_f32_dma_kernel(GemmArgs g) {
    constexpr int SA = BM * BK, SB = BK * BN, SS = SA + SB;
    constexpr int AE = A1 ? 1 : 4, BE = B1 ? 1 : 4;    // floats a lane moves per DMA
    constexpr int IAW = SA / 64 / AE / 4, IBW = SB / 64 / BE / 4;  // DMAs per wave per slab
    constexpr int KQ = BK / 4;                              // 16-byte slots per A row
    static_assert(!(A1 && TA) && !(B1 && TB) && (EDGE || !(A1 || B1)),
                  "4-byte DMA only for untransposed operands in the edge form");
    constexpr int WN_ = BN / WN, BMb = WM / 32, BNb = WN / 32;
    static_assert(SA % 1024 == 0 && SB % 1024 == 0, "whole DMA instructions per wave");
    static_assert(256 % BN == 0 || BN % 256 == 0, "B rows tile the 1 KiB pieces");
    static_assert((BM / WM) * (BN / WN) == 4, "four waves per workgroup");
    __shared__ __attribute__((aligned(16))) float smem[ST * SS];
    const int M = g.M, N = g.N, K = g.K;
    int tile;
    if (!gemm_tile(g, &tile)) return;  // padding of the grid (before any barrier)
    const int split = blockIdx.y;
    const int m0 = (tile / g.tiles_n) * BM;
    const int n0 = (tile % g.tiles_n) * BN;
    const int k_begin = split * g.k_per_split;
    const int k_len = min(g.k_per_split, K - k_begin);
    const int slabs = EDGE ? (k_len + BK - 1) / BK : k_len / BK;
    // EDGE: a last slab that K ends inside (K % 4 == 0) is loaded with the
    // pieces past K masked to zeros, as the register-staged kernel fills them
    const int tail_sl = EDGE && k_len % BK ? slabs - 1 : -1;
    const int lane = threadIdx.x & 63;
    // wave-uniform for the compiler: the DMA's LDS address (M0) is then
    // computed on the scalar unit, not by a readfirstlane per instruction
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm0 = (wave / WN_) * WM, wn0 = (wave % WN_) * WN;
    const int l32 = lane & 31, h = lane >> 5;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(g.A, (uint32_t)((size_t)M * K * 4));
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(g.B, (uint32_t)((size_t)K * N * 4));
    // this lane's DMA offsets at k = k_begin; each slab's step rides in soffset
    constexpr uint32_t kOutside = 0x80000000u;
    uint32_t aoff[IAW], boff[IBW];
    int ak[IAW], bk[IBW];  // (EDGE) the k within a slab of this lane's A and B pieces
#pragma unroll
    for (int u = 0; u < IAW; ++u) {
        const int p = (wave * IAW + u) * 64 + lane;  // AE-float position in the A stage
        if constexpr (TA) {  // k-major: row k, four m (M % 4 == 0 for EDGE)
            const int row = 4 * p / BM, col = 4 * p % BM;
            aoff[u] = ((uint32_t)(k_begin + row) * (uint32_t)M + (uint32_t)(m0 + col)) * 4u;
            if (EDGE && m0 + col >= M) aoff[u] = kOutside;
            ak[u] = row;
        } else {  // row m: 16-byte slot s holds k-piece s ^ ((m >> 2) & (KQ - 1))
            const int e = p * AE, row = e / BK, slot = (e % BK) / 4, within = e % 4;
            const int kq = slot ^ ((row >> 2) & (KQ - 1));
            aoff[u] = ((uint32_t)(m0 + row) * (uint32_t)K + (uint32_t)(k_begin + 4 * kq + within)) *
                      4u;
            if (EDGE && m0 + row >= M) aoff[u] = kOutside;
            ak[u] = 4 * kq + within;
        }
    }
#pragma unroll
    for (int u = 0; u < IBW; ++u) {
        const int p = (wave * IBW + u) * 64 + lane;  // BE-float position in the B stage
        if constexpr (TB) {  // n-major: row n, four k
            const int row = p / KQ, slot = p % KQ;
            const int kq = slot ^ ((row >> 2) & (KQ - 1));
            boff[u] = ((uint32_t)(n0 + row) * (uint32_t)K + (uint32_t)(k_begin + 4 * kq)) * 4u;
            if (EDGE && n0 + row >= N) boff[u] = kOutside;
            bk[u] = 4 * kq;
        } else {
            const int row = BE * p / BN, col = BE * p % BN;
            boff[u] = ((uint32_t)(k_begin + row) * (uint32_t)N + (uint32_t)(n0 + col)) * 4u;
            if (EDGE && n0 + col >= N) boff[u] = kOutside;
            bk[u] = row;
        }
    }
    const int a_step = TA ? BK * M * 4 : BK * 4;  // bytes per slab
    const int b_step = TB ? BK * 4 : BK * N * 4;
    auto dma = [&](int sl) {
        float *st = smem + (sl % ST) * SS;
        if (EDGE && sl == tail_sl) {  // the slab step moves into the masked offsets
            const int k0 = sl * BK;   // within this split
#pragma unroll
            for (int u = 0; u < IAW; ++u) {
                const uint32_t o = aoff[u] != kOutside && k0 + ak[u] < k_len
                                       ? aoff[u] + (uint32_t)(sl * a_step)
                                       : kOutside;
                dma_lds<A1>(ra, st + (wave * IAW + u) * 64 * AE, o, 0);
            }
#pragma unroll
            for (int u = 0; u < IBW; ++u) {
                const uint32_t o = boff[u] != kOutside && k0 + bk[u] < k_len
                                       ? boff[u] + (uint32_t)(sl * b_step)
                                       : kOutside;
                dma_lds<B1>(rb, st + SA + (wave * IBW + u) * 64 * BE, o, 0);
            }
            return;
        }
#pragma unroll
        for (int u = 0; u < IAW; ++u)
            dma_lds<A1>(ra, st + (wave * IAW + u) * 64 * AE, aoff[u], sl * a_step);
#pragma unroll
        for (int u = 0; u < IBW; ++u)
            dma_lds<B1>(rb, st + SA + (wave * IBW + u) * 64 * BE, boff[u], sl * b_step);
    };
    f16v acc[BMb][BNb];
#pragma unroll
    for (int i = 0; i < BMb; ++i)
#pragma unroll
        for (int j = 0; j < BNb; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
#pragma unroll
    for (int sl = 0; sl < ST - 1; ++sl)
        if (sl < slabs) dma(sl);
    for (int sl = 0; sl < slabs; ++sl) {
        // slab sl has landed once at most the later slabs' DMAs (IAW + IBW
        // per slab; min(ST - 2, slabs - 1 - sl) slabs) are outstanding
        static_assert(ST >= 2 && ST <= 4 && (ST - 2) * (IAW + IBW) < 64, "vmcnt range");
        const int later = min(ST - 2, slabs - 1 - sl);
        if (ST >= 4 && later >= 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * (IAW + IBW)));
        else if (ST >= 3 && later >= 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(IAW + IBW));
        else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        asm volatile("s_barrier" ::: "memory");
        if (sl + ST - 1 < slabs) dma(sl + ST - 1);
        const float *sA = smem + (sl % ST) * SS, *sB = sA + SA;
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int gk = 0; gk < BK / 8; ++gk) {
            f4 a[BMb];
            float b[BNb][4];
            const int kq = 2 * gk + h;
#pragma unroll
            for (int i = 0; i < BMb; ++i) {
                const int row = wm0 + 32 * i + l32;
                if constexpr (TA) {
#pragma unroll
                    for (int t = 0; t < 4; ++t) a[i][t] = sA[(4 * kq + t) * BM + row];
                } else {
                    a[i] = *reinterpret_cast<const f4 *>(sA + row * BK +
                                                         4 * (kq ^ ((row >> 2) & (KQ - 1))));
                }
            }
#pragma unroll
            for (int j = 0; j < BNb; ++j) {
                const int col = wn0 + 32 * j + l32;
                if constexpr (TB) {
                    const f4 v = *reinterpret_cast<const f4 *>(sB + col * BK +
                                                               4 * (kq ^ ((col >> 2) & (KQ - 1))));
#pragma unroll
                    for (int t = 0; t < 4; ++t) b[j][t] = v[t];
                } else {
#pragma unroll
                    for (int t = 0; t < 4; ++t) b[j][t] = sB[(4 * kq + t) * BN + col];
                }
            }
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int i = 0; i < BMb; ++i)
#pragma unroll
                    for (int j = 0; j < BNb; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][t], b[j][t],
                                                                         acc[i][j], 0, 0, 0);
        }
        __builtin_amdgcn_s_setprio(0);
    }
    // Accumulator element e of block (i, j) is tile element (r, c) with
    // r = wm0 + 32*i + 8*(e/4) + 4*h + e%4 and c = wn0 + 32*j + l%32.
    if (g.splits == 1) {
        float bc[BNb];  // per-column bias, loaded before any store
#pragma unroll
        for (int j = 0; j < BNb; ++j) {
            const int col = n0 + wn0 + 32 * j + l32;
            bc[j] = EPI && g.epi.bias_mode == GEMM_BIAS_COL && (!EDGE || col < N) ? g.epi.bias[col]
                                                                                   : 0.0f;
        }
        // a row's columns one after another: the row's address is live only
        // while its BNb elements are stored
#pragma unroll
        for (int i = 0; i < BMb; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e)
#pragma unroll
                for (int j = 0; j < BNb; ++j) {
                    const int row = m0 + wm0 + 32 * i + 8 * (e / 4) + 4 * h + (e % 4);
                    const int col = n0 + wn0 + 32 * j + l32;
                    const bool in = !EDGE || (row < M && col < N);
                    if constexpr (EPI) {
                        const float v =
                            epilogue(g.epi, acc_read(acc[i][j][e]), row, col, N, &bc[j]);
                        if (in) g.C[(size_t)row * N + col] = v;
                    } else {
                        if (in) g.C[(size_t)row * N + col] = acc[i][j][e];
                    }
                }
        return;
    }
    float *part = g.ws + ((size_t)split * g.tiles + tile) * (BM * BN);
#pragma unroll
    for (int i = 0; i < BMb; ++i)
#pragma unroll
        for (int j = 0; j < BNb; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int r = wm0 + 32 * i + 8 * (e / 4) + 4 * h + (e % 4);
                const int c = wn0 + 32 * j + l32;
                part[r * BN + c] = acc[i][j][e];
            }
}

// C[row][col] = sum over splits, in split order, of the parked tiles
// (deterministic).  One thread per four consecutive columns of a tile row;
// the loads of eight splits are issued before any of them is added (the
// additions stay in split order; a load-then-add loop would pay one memory
// round trip per split), and one-wave workgroups spread the few thousand
// threads over all CUs.
__global__ void __launch_bounds__(64) gemm_splitk_reduce(const float *__restrict__ ws,
                                                         float *__restrict__ C, int M, int N,
                                                         int BM, int BN, int tiles_n, int tiles,
                                                         int splits, GemmEpilogue epi) {
    const int quads_per_row = BN / 4;
    const int64_t total = (int64_t)tiles * BM * quads_per_row;
    const size_t split_stride = (size_t)tiles * BM * BN;
    for (int64_t i = (int64_t)blockIdx.x * 64 + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * 64) {
        const int tile = (int)(i / ((int64_t)BM * quads_per_row));
        const int rem = (int)(i % ((int64_t)BM * quads_per_row));
        const int r = rem / quads_per_row, c = 4 * (rem % quads_per_row);
        const int row = (tile / tiles_n) * BM + r;
        const int col = (tile % tiles_n) * BN + c;
        if (row >= M || col >= N) continue;
        const float *src = ws + (size_t)tile * BM * BN + (size_t)r * BN + c;
        constexpr int kBatch = 8;
        f4 sum = {0.f, 0.f, 0.f, 0.f};
        for (int sp0 = 0; sp0 < splits; sp0 += kBatch) {
            f4 v[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u)
                if (sp0 + u < splits)
                    v[u] = *reinterpret_cast<const f4 *>(src + (size_t)(sp0 + u) * split_stride);
#pragma unroll
            for (int u = 0; u < kBatch; ++u)  // the first split is taken as is
                if (sp0 + u < splits) sum = sp0 + u == 0 ? v[u] : sum + v[u];
        }
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (col + q < N) C[(size_t)row * N + col + q] = epilogue(epi, sum[q], row, col + q, N);
    }
}

// Skinny GEMM, M <= 32*MB (the 32-row decode-style product).
//
// With M this small, B (K x N) is almost all of the HBM traffic and every B
// element feeds at most MB MFMA steps, so the kernel is a stream over B that
// must keep the matrix cores busy at the same time: at M=32, N=K=4096 the
// MFMA floor (6.8 us) and the HBM floor (8.4 us) are close.
//  * A workgroup owns 32*NB columns of C (all M rows) and W waves; wave w
//    covers its own range of k_per_wave values of K (a K split inside the
//    workgroup); the grid's y dimension splits K further across workgroups.
//  * Column interleave: lane l (l%32 = c) loads the NB consecutive floats
//    B[k][n0 + NB*c .. NB*c + NB-1] in one load and hands float q to MFMA
//    block q, so block q computes the columns n0 + NB*c + q.  One 16-byte
//    load per lane (NB = 4) feeds four MFMA blocks, and the A values a wave
//    reads (one 16-byte load per 32-row block and 8-group of k) are shared
//    by all NB blocks: A traffic into the CU is 1/NB of B's.
//  * Each wave loads straight into the MFMA operand registers, D groups of
//    8 k ahead of the MFMAs that use them (lane half h = l/32 supplies
//    k = 8g + 4h + t, t = 0..3, as in the tiled kernel), so the loads of D
//    groups are in flight while one group is multiplied.
//  * Loads go through buffer resources: a lane's byte offset is fixed for
//    the whole wave and the per-group row step is a uniform scalar offset,
//    so there is no per-load address arithmetic.  A lane whose k lies outside
//    the wave's range (or whose row >= M / column >= N) gets an offset past
//    the end of the buffer, which the hardware answers with zeros.
//  * The W partial blocks meet in LDS and are summed in wave order
//    (deterministic), then stored through the epilogue (one split) or parked
//    for gemm_splitk_reduce, which sums the splits in order.
// Needs K % 4 == 0, N % NB == 0, a 16-byte aligned A, and A, B under 2 GiB
// each (the plan checks all four).


// Groups of 8 k values in flight per wave in the skinny kernel: two.  Deeper
// pipelines put more of B in flight at once and ran slower on every skinny
// shape measured (32x4096x4096: depth 1 20.1 us, 2 17.3 us, 4 18.6 us,
// 8 19.8 us, 16 23.5 us; 64x11008x4096: 65.4 us at depth 2, 75 us at 4 or 8).
constexpr int kSkinnyDepth = 2;

template <int NB>
__device__ __forceinline__ void load_b(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                       float *dst) {
    if constexpr (NB == 1) {
        dst[0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff,
                                                                                (int)soff, 0));
    } else if constexpr (NB == 2) {
        typedef unsigned u2 __attribute__((ext_vector_type(2)));
        const u2 v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, 0);
        dst[0] = __uint_as_float(v.x);
        dst[1] = __uint_as_float(v.y);
    } else {
        const f4 v = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff,
                                                                                  (int)soff, 0));
        dst[0] = v.x;
        dst[1] = v.y;
        dst[2] = v.z;
        dst[3] = v.w;
    }
}

template <int MB, int NB, int W, int CH>
__global__ void __launch_bounds__(64 * W) gemm_skinny_kernel(GemmArgs g) {
    constexpr int D = kSkinnyDepth;              // 8-groups in flight per wave
    constexpr int k_per_wave = 8 * D * CH;       // CH chunks of D groups
    constexpr int kRows = 32 * MB, kCols = 32 * NB;
    constexpr int kBlock = kRows * kCols;        // floats of one wave's partial tile
    __shared__ __attribute__((aligned(16))) float red[W * kBlock];
    const int M = g.M, N = g.N, K = g.K;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l32 = lane & 31, h = lane >> 5;
    const int n0 = blockIdx.x * kCols;
    const int k_begin = (blockIdx.y * W + wave) * k_per_wave;
    const int k_end = min(k_begin + k_per_wave, K);

    // The plan keeps both matrices under 2 GiB, so kOutside is past the end.
    constexpr uint32_t kOutside = 0x80000000u;
    const __amdgpu_buffer_rsrc_t rsrc_b = make_rsrc(g.B, (uint32_t)((size_t)K * N * 4));
    const __amdgpu_buffer_rsrc_t rsrc_a = make_rsrc(g.A, (uint32_t)((size_t)M * K * 4));
    const int col = n0 + NB * l32;  // first of this lane's NB columns
    const int k_lane = k_begin + 4 * h;
    const int k_lim = k_end - k_lane;  // group gi is in range iff 8*gi < k_lim
    const uint32_t boff = col < N ? ((uint32_t)k_lane * (uint32_t)N + (uint32_t)col) * 4u : kOutside;
    uint32_t aoff[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) {
        const int r = 32 * i + l32;
        aoff[i] = r < M ? ((uint32_t)r * (uint32_t)K + (uint32_t)k_lane) * 4u : kOutside;
    }
    const uint32_t row_bytes = (uint32_t)N * 4u;

    f16v acc[MB][NB];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    float bq[D][4][NB];
    f4 aq[D][MB];
    auto load = [&](int gi, int d) {
        const bool ok = 8 * gi < k_lim;  // k_end % 4 == 0, so t = 0..3 share it
        const uint32_t bv = ok ? boff : kOutside;
#pragma unroll
        for (int t = 0; t < 4; ++t) load_b<NB>(rsrc_b, bv, (uint32_t)(8 * gi + t) * row_bytes, bq[d][t]);
#pragma unroll
        for (int i = 0; i < MB; ++i)
            aq[d][i] = __builtin_bit_cast(
                f4, __builtin_amdgcn_raw_buffer_load_b128(rsrc_a, (int)(ok ? aoff[i] : kOutside),
                                                          32 * gi, 0));
    };
    auto mma = [&](int d) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < MB; ++i)
#pragma unroll
                for (int j = 0; j < NB; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(aq[d][i][t], bq[d][t][j],
                                                                     acc[i][j], 0, 0, 0);
    };

    // Rolling pipeline: consume slot d, refill it with the group D ahead.
    // The scheduling barriers keep that order (left alone, the scheduler
    // gathers each chunk's loads at its end and waits for all of them at the
    // start of the next, exposing the full load latency once per chunk).
    // The chunk loop is unrolled completely: across a loop back-edge the
    // compiler's wait counts turn conservative and drain the pipeline.
#pragma unroll
    for (int d = 0; d < D; ++d) load(d, d);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int c = 0; c + 1 < CH; ++c) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            mma(d);
            load((c + 1) * D + d, d);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
        mma(d);
        __builtin_amdgcn_sched_barrier(0);
    }

    // Accumulator element e of block (i, j) is row 32*i + 8*(e/4) + 4*h + e%4
    // and column NB*(l%32) + j of the workgroup's kCols columns.
    float *mine = red + wave * kBlock;
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            float *dst = mine + (32 * i + 8 * (e / 4) + 4 * h + (e % 4)) * kCols + NB * l32;
#pragma unroll
            for (int j = 0; j < NB; ++j) dst[j] = acc[i][j][e];
        }
    __syncthreads();

    constexpr int kPer = kBlock / (64 * W);  // consecutive outputs per thread
    static_assert(kPer >= 1 && kCols % kPer == 0, "outputs per thread split a row evenly");
    const int idx = threadIdx.x * kPer;
    float sum[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) sum[j] = red[idx + j];
    for (int w = 1; w < W; ++w)
#pragma unroll
        for (int j = 0; j < kPer; ++j) sum[j] += red[w * kBlock + idx + j];
    const int r = idx / kCols, c0 = idx % kCols;
    if (g.splits == 1) {
        if (r < M)
#pragma unroll
            for (int j = 0; j < kPer; ++j) {
                const int cc = n0 + c0 + j;
                if (cc < N) g.C[(size_t)r * N + cc] = epilogue(g.epi, sum[j], r, cc, N);
            }
        return;
    }
    float *part = g.ws + ((size_t)blockIdx.y * gridDim.x + blockIdx.x) * kBlock;
#pragma unroll
    for (int j = 0; j < kPer; ++j) part[idx + j] = sum[j];
}

// Strip path: M <= 32 with B of 4 MiB or more, in ONE launch with no
// workspace (the 32 x 4096 x 4096 decode-style product).  Every workgroup
// produces final outputs over the whole K, since a reduction across
// workgroups needs a device-scope fence per workgroup, which costs far more
// than the product on this part (+36 us at this shape, measured), or a second
// launch.  With 256 workgroups each one owns 512 outputs; a tile of 16 rows
// x 32 columns keeps its L1 fill (16 + 32 rows of K) near the minimum and
// reads B in whole 128-byte lines.  The two 16-row halves of a 32-column
// strip are neighbouring workgroups on one XCD, so the second reads B's
// lines from that XCD's L2: HBM sees B once.
//  * v_mfma_f32_16x16x4_f32 (lane l supplies A[l%16][l/16] and
//    B[l/16][l%16]; D[4(l/16) + i][l%16] in element i), two 16x16 blocks:
//    lane (l16, q) loads B[k][n0 + 2 l16 .. +1] in one 8-byte load straight
//    into operand registers, block 0 takes the even column, block 1 the odd
//    one.  kStripDepth groups of 32 k are in flight.
//  * K is split over the 4 waves (one per SIMD); a wave walks its range in
//    chunks of 64 k (two groups).  A goes through LDS: each wave keeps a ring
//    of kStripRing chunks (16 rows x 64 k, 4 KiB) filled by buffer->LDS DMA
//    (no registers) that many chunks ahead, each DMA lane moving 16
//    contiguous bytes of one row, and reads its MFMA operands from there.
//    Within a chunk, 16-byte slot s of row r holds k-piece s ^ r, so the 16
//    rows a read touches fall in different banks.  Group g + 1's A operands
//    are read from LDS while group g's MFMAs run, after an explicit vmcnt
//    wait that covers the DMA of its chunk (vector-memory operations
//    complete in issue order).
//  * Each strip starts its waves' chunk walks at a different offset
//    (strip * 3 mod chunks): the workgroups of an XCD then read different k
//    ranges of A at any moment instead of the same lines.
//  * Measured at 32 x 4096 x 4096 (cold B): A read into registers from L2,
//    16.1-17 us; A through the LDS ring, 13.1-13.8 us; a plain read of B
//    alone, 10.2 us; the split-K skinny kernel plus its reduce, 17.3-17.8 us.
//  * The 4 partial tiles meet in LDS and are summed in wave order, so the
//    result is deterministic; the epilogue applies at the store.
// A kernel variant per chunks-per-wave count NCH (the walk is unrolled: a
// loop back-edge makes the compiler's load waits conservative).  Needs
// K % 4 == 0, N % 2 == 0, a 16-byte aligned A and A, B under 2 GiB (the
// plan checks them); rows past M and k past K read as zeros (a DMA lane
// past the end of A writes zeros to LDS).
constexpr int kStripWaves = 4;
constexpr int kStripDepth = 2;   // B groups in flight
constexpr int kStripRing = 6;    // A chunks in flight per wave
constexpr int kStripRot = 3;

// FULL: K is exactly the walk (kStripWaves * 64 * NCH): no k masking, the
// row and chunk steps ride in the uniform scalar offsets.  Otherwise every
// load's offset is formed per lane and k past K is sent past the end of its
// buffer.
template <int NCH, bool EPI, bool FULL>
__global__ void __launch_bounds__(64 * kStripWaves) gemm_strip_kernel(GemmArgs g) {
    constexpr int W = kStripWaves, D = kStripDepth;
    constexpr int R = NCH < kStripRing ? NCH : kStripRing;
    constexpr int G2 = 2 * NCH;          // groups of 32 k per wave
    constexpr int CH = 16 * 64;          // floats per chunk
    constexpr int kPitch = 33;
    static_assert(R == NCH || D < 2 * R - 1, "a chunk's DMA must precede its first B group");
    __shared__ __attribute__((aligned(16))) float ring[W * R * CH];
    const int M = g.M, N = g.N, K = g.K;
    const int L = blockIdx.x;
    const int V = (L % 8) * g.per_xcd + L / 8;
    if (V >= g.tiles) return;
    const int halves = g.tiles / g.tiles_n;
    const int strip = V / halves, mh = V % halves;
    const int n0 = strip * 32, m0 = mh * 16;
    const int lane = threadIdx.x & 63;
    // wave-uniform for the compiler: the DMA's LDS address (M0) is then
    // computed on the scalar unit, not by a readfirstlane per instruction
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l16 = lane & 15, q = lane >> 4;
    const int kb = wave * (64 * NCH);
    float *myring = ring + wave * R * CH;
    // past the end of A and B (each under 2 GiB); plus any in-range offset it
    // stays below 2^32, so it never wraps back into the buffer
    constexpr uint32_t kOutside = 0x80000000u;
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(g.B, (uint32_t)((size_t)K * N * 4));
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(g.A, (uint32_t)((size_t)M * K * 4));
    const int col = n0 + 2 * l16;
    const bool col_ok = col < N;  // N is even: col + 1 < N too
    const uint32_t boff = col_ok ? ((uint32_t)(kb + 8 * q) * (uint32_t)N + (uint32_t)col) * 4u
                                 : kOutside;
    const uint32_t row_bytes = (uint32_t)N * 4u;
    // DMA lane mapping: instruction j, lane l -> chunk row 4j + l/16, slot
    // l%16, holding k-piece slot ^ row.  Rows >= M start at or past M * K * 4,
    // the end of A.
    uint32_t adma[4];
    int akp[4];  // this lane's k offset within a chunk, per instruction
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int row = 4 * j + (lane >> 4), slot = lane & 15;
        akp[j] = 4 * (slot ^ row);
        adma[j] = ((uint32_t)(m0 + row) * (uint32_t)K + (uint32_t)(kb + akp[j])) * 4u;
    }
    const int rot = (strip * kStripRot) % NCH;
    auto dma = [&](int c0) {  // chunk c0 of the walk into its ring slot
        const int c = (c0 + rot) % NCH;
        float *dst = myring + (c0 % R) * CH;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (FULL) {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void *)(dst + 256 * j), 16,
                                                         (int)adma[j], 256 * c, 0, 0);
            } else {
                // past K a row would run on into the next one
                const uint32_t o = kb + 64 * c + akp[j] < K ? adma[j] + 256u * c : kOutside;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void *)(dst + 256 * j), 16, (int)o,
                                                         0, 0, 0);
            }
        }
    };
    typedef unsigned u2 __attribute__((ext_vector_type(2)));
    float bq[D][8][2];
    auto loadb = [&](int g0, int d) {  // group g0 of the walk
        const int gi = 2 * (((g0 >> 1) + rot) % NCH) + (g0 & 1);
        const int k0 = kb + 32 * gi + 8 * q;  // this lane's first k of the group
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            u2 v;
            if (FULL) {
                v = __builtin_amdgcn_raw_buffer_load_b64(
                    rb, (int)boff, (int)((uint32_t)(32 * gi + t) * row_bytes), 0);
            } else {
                const uint32_t o = (col_ok && k0 + t < K)
                                       ? boff + (uint32_t)(32 * gi + t) * row_bytes
                                       : kOutside;
                v = __builtin_amdgcn_raw_buffer_load_b64(rb, (int)o, 0, 0);
            }
            bq[d][t][0] = __uint_as_float(v.x);
            bq[d][t][1] = __uint_as_float(v.y);
        }
    };
    f4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    // A operands of two groups (slot g & 1): group g + 1's are read from LDS
    // while group g's MFMAs run, so the LDS latency is hidden behind them
    f4 aop[2][2];
    auto read_a = [&](int g0) {
        const float *src = myring + ((g0 >> 1) % R) * CH + l16 * 64;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            // lane (l16, q) covers k = 32 sg + 8q + 4h + (0..3) of the chunk
            const int piece = 8 * (g0 & 1) + 2 * q + h;
            aop[g0 & 1][h] = *reinterpret_cast<const f4 *>(src + 4 * (piece ^ l16));
        }
    };
    auto mma = [&](int g0, int d) {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const float a = aop[g0 & 1][t / 4][t % 4];
            acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a, bq[d][t][0], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a, bq[d][t][1], acc1, 0, 0, 0);
        }
    };
    // Issue order (the counts below follow from it; sched_barrier keeps the
    // regions in order): prologue = DMA of chunk 0, the first D B groups, the
    // DMA of chunks 1 .. R-1; region gi = B group gi + D and, for odd gi, the
    // DMA of chunk gi/2 + R.  Before group g's A operands are read from LDS, an explicit
    // vmcnt wait leaves outstanding only the vector-memory operations issued
    // after the DMA of g's chunk (those operations, the LDS DMAs included,
    // complete in issue order), so the read never sees a stale ring slot.
    // The DMA went out several groups earlier, so the wait rarely stalls;
    // the B operands are waited for register by register by the compiler,
    // so a group's MFMAs start as its first loads arrive.
    constexpr int kB = 8, kDma = 4;  // vector-memory instructions per B group / chunk DMA
    auto dma_in = [&](int j) {       // DMA instructions of region j
        return ((j & 1) && j / 2 + R < NCH) ? kDma : 0;
    };
    auto region = [&](int j) { return (j + D < G2 ? kB : 0) + dma_in(j); };
    // operations issued after chunk c's DMA, up to the start of region gi
    auto after_dma = [&](int c, int gi) {
        int n = 0;
        if (c < R) {
            n = kDma * (R - 1 - c);
            if (c == 0)
                for (int g = 0; g < D && g < G2; ++g) n += kB;
            for (int j = 0; j < gi; ++j) n += region(j);
        } else {
            // region 2(c - R) + 1 issued it; its own B loads may follow it
            for (int j = 2 * (c - R) + 1; j < gi; ++j) n += region(j);
        }
        return n;
    };
    dma(0);
#pragma unroll
    for (int d = 0; d < D && d < G2; ++d) loadb(d, d);
#pragma unroll
    for (int c = 1; c < R; ++c) dma(c);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int gi = 0; gi < G2; ++gi) {
        // group gi + 1's A operands (group 0's too, on the first pass): its
        // chunk's DMA must be complete; 63 or more later operations imply it
        const int next = gi + 1 < G2 ? gi + 1 : gi;
        const int n = after_dma(next >> 1, gi);
        if (n < 63) wait_vmem(n);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        if (gi == 0) read_a(0);
        if (gi + 1 < G2) read_a(gi + 1);
        __builtin_amdgcn_sched_barrier(0);  // the reads go out before the MFMAs
        mma(gi, gi % D);
        if (gi + D < G2) loadb(gi + D, gi % D);
        // the slot of chunk gi/2 is free: both its groups' operands are in
        // registers (the MFMAs above waited for group gi's reads)
        if ((gi & 1) && gi / 2 + R < NCH) dma(gi / 2 + R);
        __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();  // every wave is done with its ring: reuse it for the sums
    // lane holds rows 4q + j: block 0 at column 2 l16, block 1 at 2 l16 + 1
    float *red = ring;
    float *mine = red + wave * 16 * kPitch;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        mine[(4 * q + j) * kPitch + 2 * l16] = acc0[j];
        mine[(4 * q + j) * kPitch + 2 * l16 + 1] = acc1[j];
    }
    __syncthreads();
    // 512 outputs over 256 threads, each summed in wave order
    for (int o = threadIdx.x; o < 16 * 32; o += 64 * W) {
        const int r = o / 32, c = o % 32;
        float sum = red[r * kPitch + c];
#pragma unroll
        for (int w = 1; w < W; ++w) sum += red[w * 16 * kPitch + r * kPitch + c];
        const int gr = m0 + r, gc = n0 + c;
        if (gr < M && gc < N)
            g.C[(size_t)gr * N + gc] = EPI ? epilogue(g.epi, sum, gr, gc, N) : sum;
    }
}

// Small path: products whose tiles of 16*MB x 16 fit the chip in one wave
// of workgroups and whose K is at most 1024 (the MLP layers, decode-sized
// projections).  Every tile of C gets one workgroup of W waves that
// splits K inside the workgroup: wave w covers [w * kpw, (w + 1) * kpw) and
// builds a full partial tile on v_mfma_f32_16x16x4_f32 straight from global
// memory, and the W partials meet in LDS and are summed in wave order.  No
// workspace and no second kernel, where a split across workgroups needs a
// reduce launch; the sum is deterministic for a given shape.  16-column
// tiles give four times the workgroups of 32-column ones: a 64 x 128
// product still spreads over 32 CUs.
//
// Operand layout of v_mfma_f32_16x16x4_f32: lane l supplies A[l%16][l/16]
// and B[l/16][l%16] and holds D[4(l/16) + i][l%16] in accumulator element i.
// A K-group of 16 is split as k = 16g + 4q + t: lane group q = l/16 reads
// its four k values of A in one 16-byte load per 16-row block, MFMA step t
// consumes component t, and B is read one float per lane and step (16
// columns x 4 rows per load).  A wave's K range is NBATCH batches of four
// groups (64 k; the plan uses one); the loads of batch b + 1 are issued
// before batch b's MFMAs, and the batches are unrolled, so every wait drains
// only the older batch.  Out-of-range groups load zeros through offsets past
// the buffer.
//
// Tile order: workgroup L takes position (L % 8) * ceil(tiles / 8) + L / 8,
// so each XCD (workgroups are dealt to the 8 XCDs round-robin) owns a run of
// adjacent column strips whose 64-byte row pieces share 128-byte lines in
// its L2.
// Needs K % 4 == 0, a 16-byte aligned A and A, B under 2 GiB (the plan
// checks them).
template <int MB>
struct SmallBatch {
    f4 a[4][MB];
    float b[4][4];
};

// One tile V of product g (the body of the small-path kernels).
template <int W, int MB, int NBATCH, bool EPI>
__device__ __forceinline__ void small_tile(const GemmArgs &g, int V) {
    constexpr int kRows = 16 * MB;
    constexpr int kPitch = 17;
    __shared__ float red[W * kRows * kPitch];
    const int M = g.M, N = g.N, K = g.K;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l16 = lane & 15, q = lane >> 4;
    const int m0 = (V / g.tiles_n) * kRows, n0 = (V % g.tiles_n) * 16;
    const int kpw = g.k_per_split;  // 64 * NBATCH
    const int kb = wave * kpw;
    const int ke = min(kb + kpw, K);
    constexpr uint32_t kOutside = 0x80000000u;
    const __amdgpu_buffer_rsrc_t rsrc_a = make_rsrc(g.A, (uint32_t)((size_t)M * K * 4));
    const __amdgpu_buffer_rsrc_t rsrc_b = make_rsrc(g.B, (uint32_t)((size_t)K * N * 4));
    const int col = n0 + l16;
    const int k_lane = kb + 4 * q;
    uint32_t aoff[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) {
        const int row = m0 + 16 * i + l16;
        aoff[i] = row < M && k_lane < K ? ((uint32_t)row * (uint32_t)K + (uint32_t)k_lane) * 4u
                                        : kOutside;
    }
    const uint32_t boff = col < N && k_lane < K ? ((uint32_t)k_lane * (uint32_t)N + (uint32_t)col) * 4u
                                                : kOutside;
    const uint32_t row_bytes = (uint32_t)N * 4u;
    const int groups = ke > kb ? (ke - kb + 15) / 16 : 0;

    // group gi is in range for lane group q iff k = kb + 16gi + 4q (and the
    // next three, K % 4 == 0) is below ke
    auto load = [&](int g0, SmallBatch<MB> &x) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const int gi = g0 + d;
            const bool ok = gi < groups && kb + 16 * gi + 4 * q < ke;
#pragma unroll
            for (int i = 0; i < MB; ++i)
                x.a[d][i] = __builtin_bit_cast(
                    f4, __builtin_amdgcn_raw_buffer_load_b128(
                            rsrc_a, (int)(ok ? aoff[i] : kOutside), 64 * gi, 0));
#pragma unroll
            for (int t = 0; t < 4; ++t)
                x.b[d][t] = __builtin_bit_cast(
                    float, __builtin_amdgcn_raw_buffer_load_b32(
                               rsrc_b, (int)(ok ? boff : kOutside),
                               (int)((uint32_t)(16 * gi + t) * row_bytes), 0));
        }
    };
    f4 acc[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) acc[i] = (f4){0.f, 0.f, 0.f, 0.f};
    SmallBatch<MB> buf[2];
    load(0, buf[0]);
#pragma unroll
    for (int bi = 0; bi < NBATCH; ++bi) {
        if (bi + 1 < NBATCH) load(4 * (bi + 1), buf[(bi + 1) & 1]);
        // keep each batch whole and ahead of the previous batch's MFMAs
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int i = 0; i < MB; ++i)
                    acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(buf[bi & 1].a[d][i][t],
                                                                  buf[bi & 1].b[d][t], acc[i], 0,
                                                                  0, 0);
        __builtin_amdgcn_sched_barrier(0);
    }

    float *mine = red + wave * kRows * kPitch;
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) mine[(16 * i + 4 * q + e) * kPitch + l16] = acc[i][e];
    __syncthreads();
    if (EPI && g.epi.act == GEMM_ACT_SOFTMAX) {
        // The tile holds whole rows (N <= 16: the host only asks for this
        // epilogue then).  Bias first, rounded as the separate Add would,
        // then each row's softmax as the row kernel computes it: max, 2^x
        // exponentials of (x - max) * log2 e, their sum, one reciprocal.
        __shared__ float rowv[kRows][17];
        GemmEpilogue eb = g.epi;
        eb.act = GEMM_ACT_NONE;
        for (int idx = threadIdx.x; idx < kRows * 16; idx += 64 * W) {
            const int r = idx / 16, c = idx % 16;
            float sum = red[r * kPitch + c];
#pragma unroll
            for (int w = 1; w < W; ++w) sum += red[w * kRows * kPitch + r * kPitch + c];
            rowv[r][c] = c < N ? epilogue(eb, sum, m0 + r, c, N) : -INFINITY;
        }
        __syncthreads();
        const int r = threadIdx.x, gr = m0 + r;
        if (r < kRows && gr < M) {
            float mx = -INFINITY;
            for (int c = 0; c < N; ++c) mx = fmaxf(mx, rowv[r][c]);
            float se = 0.0f;
            for (int c = 0; c < N; ++c) {
                rowv[r][c] = __builtin_amdgcn_exp2f((rowv[r][c] - mx) * 1.44269504088896341f);
                se += rowv[r][c];
            }
            const float inv = 1.0f / se;
            for (int c = 0; c < N; ++c) g.C[(size_t)gr * N + c] = rowv[r][c] * inv;
        }
        return;
    }
    for (int idx = threadIdx.x; idx < kRows * 16; idx += 64 * W) {
        const int r = idx / 16, c = idx % 16;
        float sum = red[r * kPitch + c];
#pragma unroll
        for (int w = 1; w < W; ++w) sum += red[w * kRows * kPitch + r * kPitch + c];
        const int gr = m0 + r, gc = n0 + c;
        if (gr < M && gc < N)
            g.C[(size_t)gr * N + gc] = EPI ? epilogue(g.epi, sum, gr, gc, N) : sum;
    }
}

template <int W, int MB, int NBATCH, bool EPI>
__global__ void __launch_bounds__(64 * W) gemm_small_kernel(GemmArgs g) {
    const int L = blockIdx.x;
    const int V = (L % 8) * g.per_xcd + L / 8;
    if (V >= g.tiles) return;
    small_tile<W, MB, NBATCH, EPI>(g, V);
}

// Grouped form (the planner's horizontal MatMul groups): one launch covers
// the tiles of up to kGemmGroupMax independent small-path products; workgroup
// L runs tile L - starts[p] of the product p whose range holds it.  The
// waves per workgroup are the largest any member needs (members with a
// shorter K leave the extra waves' K ranges empty), one row block per tile.
struct GroupedArgs {
    GemmArgs prob[kGemmGroupMax];
    int starts[kGemmGroupMax + 1];
    int count;
};

template <int W>
__global__ void __launch_bounds__(64 * W) gemm_small_grouped_kernel(GroupedArgs ga) {
    const int L = blockIdx.x;
    int p = 0;
    while (p + 1 < ga.count && L >= ga.starts[p + 1]) ++p;
    small_tile<W, 1, 1, true>(ga.prob[p], L - ga.starts[p]);
}

// K = 0: C = epilogue(0) (bias and activation still apply).  A kernel rather
// than a memset, so a caller capturing the stream into a graph records no
// memset node.
__global__ void __launch_bounds__(256) gemm_k0_kernel(float *__restrict__ C, int M, int N,
                                                      GemmEpilogue epi) {
    const uint64_t total = (uint64_t)M * N;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < total;
         i += (uint64_t)gridDim.x * 256)
        C[i] = epilogue(epi, 0.0f, (int)(i / N), (int)(i % N), N);
}

// Tile configurations: (BM, BN, BK, WM, WN).
enum { CFG_32x128 = 0, CFG_64x64 = 1, CFG_128x128 = 2, CFG_128x128_K32 = 3, CFG_256x128 = 4,
       CFG_128x256 = 5, CFG_64x128 = 6, CFG_COUNT = 7 };
const int kCfgBM[CFG_COUNT] = {32, 64, 128, 128, 256, 128, 64};
const int kCfgBN[CFG_COUNT] = {128, 64, 128, 128, 128, 256, 128};
const int kCfgBK[CFG_COUNT] = {32, 16, 16, 32, 16, 16, 16};

// Whether the DMA-staged kernel takes a plan: interior tiles of the 128 x 256,
// 128 x 128 and 64 x 128 configurations with A and B under 2 GiB (32-bit
// buffer offsets).  CLOVE_GEMM_DMA=0 keeps the register-staged kernel (tests).
bool dma_ok(const GemmPlan &p, int BM, int BN) {
    const char *v = std::getenv("CLOVE_GEMM_DMA");
    const bool enabled = !(v && *v && std::atoi(v) == 0);
    return enabled && p.interior && ((BM == 128 && (BN == 256 || BN == 128)) || (BM == 64 && BN == 128)) &&
           (uint64_t)p.M * p.K * 4 < (1ull << 31) && (uint64_t)p.K * p.N * 4 < (1ull << 31);
}

// The same for tiles reaching past M or N, or K ending inside a slab:
// 16-byte aligned rows (p.vec after the pointer check: K % 4 == N % 4 == 0)
// and every split but the last a whole number of 16-deep slabs.
bool dma_edge_ok(const GemmPlan &p, int BM, int BN) {
    const char *v = std::getenv("CLOVE_GEMM_DMA");
    const bool enabled = !(v && *v && std::atoi(v) == 0);
    return enabled && !p.interior && p.vec && ((BM == 128 && (BN == 256 || BN == 128)) || (BM == 64 && BN == 128)) &&
           p.k_per_split % 16 == 0 && (uint64_t)p.M * p.K * 4 < (1ull << 31) &&
           (uint64_t)p.K * p.N * 4 < (1ull << 31);
}

// Rows that are not 16-byte aligned (K or N not a multiple of 4, or an
// operand that starts off a 16-byte boundary) in 128x128 or 64x128 tiles:
// the edge form with that operand moved one float a lane.
bool dma_odd_ok(const GemmPlan &p, int BM, int BN) {
    const char *v = std::getenv("CLOVE_GEMM_DMA");
    const bool enabled = !(v && *v && std::atoi(v) == 0);
    return enabled && !p.vec && BN == 128 && (BM == 128 || BM == 64) &&
           p.k_per_split % 16 == 0 && (uint64_t)p.M * p.K * 4 < (1ull << 31) &&
           (uint64_t)p.K * p.N * 4 < (1ull << 31);
}

template <int BM, int BN, int BK, int WM, int WN, int ST, bool EPI>
void launch_dma_odd(bool a1, bool b1, dim3 grid, const GemmArgs &g, hipStream_t s) {
    if (a1 && b1)
        gemm_f32_dma_kernel<BM, BN, BK, WM, WN, EPI, false, false, ST, true, true, true>
            <<<grid, 256, 0, s>>>(g);
    else if (a1)
        gemm_f32_dma_kernel<BM, BN, BK, WM, WN, EPI, false, false, ST, true, true, false>
            <<<grid, 256, 0, s>>>(g);
    else
        gemm_f32_dma_kernel<BM, BN, BK, WM, WN, EPI, false, false, ST, true, false, true>
            <<<grid, 256, 0, s>>>(g);
}

template <int BM, int BN, int BK, int WM, int WN>
void launch_cfg(const GemmPlan &p, GemmArgs g, hipStream_t s) {
    const dim3 grid((unsigned)(g.per_xcd * 8), (unsigned)p.splits);
    // The fused epilogue (bias modulo, GELU) costs registers; kernels without
    // one (and split-K kernels, whose reduce applies it) are built without it.
    const bool epi = p.splits == 1 &&
                     (g.epi.bias_mode != GEMM_BIAS_NONE || g.epi.act != GEMM_ACT_NONE);
    if constexpr (((BM == 128 && (BN == 256 || BN == 128)) || (BM == 64 && BN == 128)) && BK == 16) {
        constexpr int ST = dma_stages(BN);
        if (dma_ok(p, BM, BN)) {
            if (epi)
                gemm_f32_dma_kernel<BM, BN, BK, WM, WN, true, false, false, ST><<<grid, 256, 0, s>>>(g);
            else
                gemm_f32_dma_kernel<BM, BN, BK, WM, WN, false, false, false, ST><<<grid, 256, 0, s>>>(g);
            return;
        }
        if (dma_edge_ok(p, BM, BN)) {
            if (epi)
                gemm_f32_dma_kernel<BM, BN, BK, WM, WN, true, false, false, ST, true>
                    <<<grid, 256, 0, s>>>(g);
            else
                gemm_f32_dma_kernel<BM, BN, BK, WM, WN, false, false, false, ST, true>
                    <<<grid, 256, 0, s>>>(g);
            return;
        }
        if constexpr (BN == 128) {
            if (dma_odd_ok(p, BM, BN)) {
                const bool a1 = p.K % 4 != 0 || (reinterpret_cast<uintptr_t>(g.A) & 15) != 0;
                const bool b1 = p.N % 4 != 0 || (reinterpret_cast<uintptr_t>(g.B) & 15) != 0;
                if (epi)
                    launch_dma_odd<BM, BN, BK, WM, WN, ST, true>(a1, b1, grid, g, s);
                else
                    launch_dma_odd<BM, BN, BK, WM, WN, ST, false>(a1, b1, grid, g, s);
                return;
            }
        }
    }
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

template <int MB, int NB, int W>
void launch_skinny_w(const GemmPlan &p, const GemmArgs &g, dim3 grid, hipStream_t s) {
    constexpr int chunk = 8 * kSkinnyDepth;      // k per chunk of pipeline groups
    switch (p.k_per_wave / chunk) {
    case 1: gemm_skinny_kernel<MB, NB, W, 1><<<grid, 64 * W, 0, s>>>(g); break;
    case 2: gemm_skinny_kernel<MB, NB, W, 2><<<grid, 64 * W, 0, s>>>(g); break;
    case 4: gemm_skinny_kernel<MB, NB, W, 4><<<grid, 64 * W, 0, s>>>(g); break;
    case 8: gemm_skinny_kernel<MB, NB, W, 8><<<grid, 64 * W, 0, s>>>(g); break;
    default: gemm_skinny_kernel<MB, NB, W, 16><<<grid, 64 * W, 0, s>>>(g); break;
    }
}

// (mb, nb, waves) variants: LDS holds waves * 32mb x 32nb floats (<= 64 KiB).
void launch_skinny(const GemmPlan &p, const GemmArgs &g, dim3 grid, hipStream_t s) {
    if (p.mb == 1 && p.nb == 4) launch_skinny_w<1, 4, 4>(p, g, grid, s);
    else if (p.mb == 1 && p.nb == 2) launch_skinny_w<1, 2, 8>(p, g, grid, s);
    else if (p.mb == 1) launch_skinny_w<1, 1, 8>(p, g, grid, s);
    else if (p.nb == 2) launch_skinny_w<2, 2, 4>(p, g, grid, s);
    else launch_skinny_w<2, 1, 8>(p, g, grid, s);
}

template <int NCH>
void launch_strip_g(const GemmArgs &g, hipStream_t s) {
    const bool epi = g.epi.bias_mode != GEMM_BIAS_NONE || g.epi.act != GEMM_ACT_NONE;
    const bool full = g.K == kStripWaves * 64 * NCH;
    const unsigned grid = (unsigned)(8 * g.per_xcd);
    if (epi && full) gemm_strip_kernel<NCH, true, true><<<grid, 64 * kStripWaves, 0, s>>>(g);
    else if (epi) gemm_strip_kernel<NCH, true, false><<<grid, 64 * kStripWaves, 0, s>>>(g);
    else if (full) gemm_strip_kernel<NCH, false, true><<<grid, 64 * kStripWaves, 0, s>>>(g);
    else gemm_strip_kernel<NCH, false, false><<<grid, 64 * kStripWaves, 0, s>>>(g);
}

void launch_strip(const GemmPlan &p, const GemmArgs &g, hipStream_t s) {
    switch (p.k_per_wave / 64) {
    case 1: launch_strip_g<1>(g, s); break;
    case 2: launch_strip_g<2>(g, s); break;
    case 4: launch_strip_g<4>(g, s); break;
    case 8: launch_strip_g<8>(g, s); break;
    case 16: launch_strip_g<16>(g, s); break;
    case 32: launch_strip_g<32>(g, s); break;
    default: launch_strip_g<64>(g, s); break;
    }
}

template <int W, int MB, int NBATCH>
void launch_small_b(const GemmPlan &p, const GemmArgs &g, hipStream_t s) {
    const bool epi = g.epi.bias_mode != GEMM_BIAS_NONE || g.epi.act != GEMM_ACT_NONE;
    const unsigned grid = (unsigned)(8 * g.per_xcd);
    if (epi) gemm_small_kernel<W, MB, NBATCH, true><<<grid, 64 * W, 0, s>>>(g);
    else gemm_small_kernel<W, MB, NBATCH, false><<<grid, 64 * W, 0, s>>>(g);
}

template <int MB>
void launch_small_m(const GemmPlan &p, const GemmArgs &g, hipStream_t s) {
    switch (p.waves) {
    case 2: launch_small_b<2, MB, 1>(p, g, s); return;
    case 4: launch_small_b<4, MB, 1>(p, g, s); return;
    case 8: launch_small_b<8, MB, 1>(p, g, s); return;
    default: launch_small_b<16, MB, 1>(p, g, s); return;
    }
}

void launch_small(const GemmPlan &p, const GemmArgs &g, hipStream_t s) {
    if (p.mb == 1) launch_small_m<1>(p, g, s);
    else if (p.mb == 2) launch_small_m<2>(p, g, s);
    else launch_small_m<4>(p, g, s);
}

}  // namespace

// Tile shape and K split above 64 rows, for operands under 2 GiB (the DMA
// kernels' limit).  Each candidate (128x128 or 64x128 tiles, K split s ways)
// is priced as its padded MFMA work over how evenly its workgroups fill the
// CUs and an occupancy factor, plus a split's reduce pass (the partial tiles
// written and read back, the result written, one more launch):
//  * balance u / ceil(u), u = workgroups per CU: a CU's share comes in whole
//    workgroups, so 2.25 per CU takes as long as 3;
//  * one workgroup alone on a CU waits on its own loads and barriers (x0.85
//    for 128x128; x0.80 for 64x128, whose waves hold half the MFMA work
//    each), and 64x128 tiles still trail at two per CU (x0.95);
//  * 128x128 tiles are preferred by 2% where the rest ties.
// Against the fixed rule it replaces (128x128 tiles, split only below two
// per CU), measured in TFLOP/s with HIP events: 2048^3 122 -> 130, 2100^3
// 91 -> 112, 2560^3 106 -> 121, 2900^3 92 -> 116, 1536^3 88 -> 100,
// 768x4096x4096 100 -> 126, 4096x1024x1024 109 -> 125, 16384x784x128
// 81 -> 101, 3500x700x2900 107 -> 124; 37 shapes in all took 5.5% less time
// and none lost more than 0.9%.  Shapes that fill the chip evenly keep
// unsplit 128x128 tiles (4096^3, 3072x4096x4096, 2048x4096x4096).
struct TileChoice {
    int cfg, splits;
};

// only64: price 64x128 tiles alone (33-64 rows, where 128-row tiles waste
// half their work).
static TileChoice choose_tiles(int M, int N, int K, int num_cus, bool only64 = false) {
    constexpr double kMfma = 1.4e14;  // sustained FP32 MFMA FLOP/s
    constexpr double kHbm = 8e12;     // bytes/s
    constexpr double kLaunch = 3e-6;  // a second launch, s
    static const int kSplits[] = {1, 2, 3, 4, 6, 8, 12, 16, 24, 32, 48, 64};
    const int slabs = (K + 15) / 16;  // BK = 16 in both configurations
    TileChoice best{CFG_128x128, 1};
    double best_t = 0.0;
    for (const int cfg : {CFG_128x128, CFG_64x128}) {
        if (only64 && cfg != CFG_64x128) continue;
        const int BM = kCfgBM[cfg], BN = kCfgBN[cfg];
        const int64_t tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
        for (const int s : kSplits) {
            if (s > 1 && s > slabs / 4) break;  // at least four slabs per split
            const int per = (slabs + s - 1) / s;
            const int made = (slabs + per - 1) / per;
            const double u = (double)(tm * tn * made) / num_cus;
            const double bal = u / std::ceil(u);
            double occ = 1.0;
            if (u <= 1.0) occ = cfg == CFG_128x128 ? 0.85 : 0.80;
            else if (u <= 2.0 && cfg == CFG_64x128) occ = 0.95;
            const double pref = cfg == CFG_128x128 ? 1.02 : 1.0;
            const double work = 2.0 * (double)(tm * BM) * (double)(tn * BN) * (double)made *
                                (double)per * 16.0;
            double t = work / kMfma / (bal * occ * pref);
            if (made > 1) t += (2.0 * made + 1.0) * 4.0 * (double)M * (double)N / kHbm + kLaunch;
            if (best_t == 0.0 || t < best_t) {
                best_t = t;
                best = {cfg, made};
            }
        }
    }
    return best;
}

GemmPlan gemm_plan(int M, int N, int K, int num_cus, int force_cfg, bool a_aligned,
                   bool force_skinny, int force_skinny_nb, int force_skinny_splits,
                   bool force_strip, bool b_aligned) {
    GemmPlan p{};
    p.M = M;
    p.N = N;
    p.K = K;
    if (M <= 0 || N <= 0 || K <= 0) {  // nothing to tile: gemm_f32 returns at
        p.tiles = p.tiles_n = 1;         // once or (K = 0) writes epilogue(0)
        p.splits = 1;
        return p;
    }
    // Skinny path: M <= 64 (one or two 32-row blocks per wave), K % 4 == 0,
    // a 16-byte aligned A and B under 2 GiB.  NB column blocks per wave: 4
    // for M <= 32, 2 for M <= 64, fewer when N is not a multiple.  It is
    // chosen for a B of 4 MiB and more: there it measured ahead of the tiled
    // kernel (M=32, N=K=4096: 17.3 against 19.4 us, reduce included); on
    // small B the tiled split-K kernel finishes first (more parallelism per
    // MFMA chain), so the skinny path runs there only when forced.
    const uint64_t b_bytes = (uint64_t)K * (uint64_t)N * 4u;
    // Small path: when tiles of 16*mb x 16 fit the chip in one wave of
    // workgroups and K <= 1024, split K inside one workgroup per tile (no
    // workspace, one launch) instead of across workgroups with a reduce
    // launch.  mb is the fewest row blocks (1, 2, 4) whose tiles fit, so the
    // work spreads over as many CUs as possible.  2-16 waves, one batch of at
    // most 64 k each.  Longer K keeps the tiled or skinny split-K forms, which
    // spread it over every CU (at M = 32, N = K = 4096 this path with 16
    // waves and 4 batches per wave measured 22.1 us against the skinny
    // kernel's 19.2 us).
    {
        int mb = 1;
        auto tiles_for = [&](int b) { return ((M + 16 * b - 1) / (16 * b)) * ((N + 15) / 16); };
        while (mb < 4 && tiles_for(mb) > num_cus) mb *= 2;
        const int tiles = tiles_for(mb);
        if (force_cfg < 0 && !force_skinny && K >= 4 && K % 4 == 0 && K <= 1024 && a_aligned &&
            tiles <= num_cus && b_bytes < (1ull << 31) && (uint64_t)M * K * 4 < (1ull << 31)) {
            p.small = true;
            p.mb = mb;
            int w = 2;
            while (w < 16 && w * 64 < K) w *= 2;
            p.waves = w;
            p.k_per_split = 64;
            p.tiles_n = (N + 15) / 16;
            p.tiles = tiles;
            p.splits = 1;
            p.ws_floats = 0;
            p.vec = true;
            return p;
        }
    }
    const bool eligible = M <= 64 && K >= 4 && K % 4 == 0 && a_aligned && b_aligned &&
                          b_bytes < (1ull << 31) && (uint64_t)M * K * 4 < (1ull << 31) &&
                          force_cfg < 0;
    // Strip path (one launch, no workspace; M <= 32, even N, K within the
    // longest unrolled walk of 4 waves x 64 chunks of 64 k): only when forced
    // (CLOVE_GEMM_STRIP).  Only one of each strip's two 16-row halves pulls
    // B from HBM (the other reads it from its XCD's L2), so 128 workgroups
    // carry the read: with B cycled through copies that the 256 MB
    // last-level cache cannot hold, as a decode step's weights are,
    // the skinny kernel is ahead at every shape measured (1, 8, 32 x 4096 x
    // 4096: 19.0, 19.8, 21.5 us against 20.6, 22.7, 23.3; 32 x 4096 x 11008:
    // 49.0 against 61.3).  The strip kernel led only while B stayed in that
    // cache (32 x 4096 x 4096: 13.8 against 17.3 us).
    {
        const int halves = (M + 15) / 16, strips = (N + 31) / 32;
        int nch = 1;
        while (nch < 64 && kStripWaves * 64 * nch < K) nch *= 2;
        if (eligible && !force_skinny && M <= 32 && N % 2 == 0 && K <= kStripWaves * 64 * 64 &&
            force_strip) {
            p.strip = true;
            p.tiles_n = strips;
            p.tiles = halves * strips;
            p.k_per_wave = 64 * nch;
            p.waves = kStripWaves;
            p.splits = 1;
            p.ws_floats = 0;
            p.vec = true;
            return p;
        }
    }
    // 33-64 rows over a long K (and N >= 2048, whole 16-byte pieces): 64x128
    // DMA-staged tiles split over K run ahead of the skinny kernel, whose
    // per-wave chains grow with K: 64x14336x4096 80.2 against 103.3 us,
    // 64x8192x8192 89.8 against 110.5, 48x11008x4096 63.0 against 73.5; at
    // K = 4096 the skinny kernel stays ahead (64x4096x4096 28.5 against
    // 30.4 us), as it does for N = 1024.
    // The same tiles win for 33-64 rows over a vocabulary-sized N (any
    // alignment, on the 4-byte DMA form where N % 4 != 0): 64 x 4096 x 50256
    // 279 against 308 us, 40 x 4096 x 32000 149 against 163, 36 x 4096 x 50257
    // 317 against 346 (48 x 4096 x 50256 a tie; at N = 14336 the skinny
    // kernel stays ahead, 75.5 against 84.1).
    const bool long_k64 = eligible && !force_skinny && M > 32 &&
                          ((K > 4096 && N >= 2048 && N % 4 == 0) || N >= 30000);
    if (eligible && !long_k64 && (force_skinny || b_bytes >= (4ull << 20))) {
        p.skinny = true;
        p.mb = M <= 32 ? 1 : 2;
        int nb = p.mb == 1 ? 4 : 2;
        if (force_skinny_nb == 1 || force_skinny_nb == 2 || (force_skinny_nb == 4 && p.mb == 1))
            nb = force_skinny_nb;
        // (four 4-byte loads a lane for N % 4 != 0, keeping four column
        // blocks, measured no faster: 16 x 4096 x 50257 243 us against 248)
        while (nb > 1 && N % nb != 0) nb /= 2;
        p.nb = nb;
        p.waves = (nb == 1 || (nb == 2 && p.mb == 1)) ? 8 : 4;
        const int W = p.waves;
        const int chunk = 8 * kSkinnyDepth;
        p.tiles_n = (N + 32 * nb - 1) / (32 * nb);
        p.tiles = p.tiles_n;
        // Splits: enough workgroups for every CU and one wave per SIMD
        // (measured at M=32, N=K=4096: 8 splits of 4-wave groups beat 16;
        // more waves per SIMD did not help).
        int splits = (4 * num_cus + p.tiles * W - 1) / (p.tiles * W);
        const int for_cus = (num_cus + p.tiles - 1) / p.tiles;
        if (splits < for_cus) splits = for_cus;
        const int max_splits = K / (chunk * W) > 1 ? K / (chunk * W) : 1;
        if (splits > max_splits) splits = max_splits;
        if (force_skinny_splits > 0) splits = force_skinny_splits;
        if (splits > 64) splits = 64;
        if (splits < 1) splits = 1;
        // k_per_wave is chunk * CH for CH in {1, 2, 4, 8, 16} (kernel variants);
        // a longer range takes more splits instead.
        const int kw_raw = (K + splits * W - 1) / (splits * W);
        int ch = 1;
        while (ch < 16 && chunk * ch < kw_raw) ch *= 2;
        p.k_per_wave = chunk * ch;
        p.k_per_split = p.k_per_wave * W;
        p.splits = (K + p.k_per_split - 1) / p.k_per_split;
        p.ws_floats = p.splits > 1 ? (size_t)p.splits * p.tiles * (32 * p.mb) * (32 * nb) : 0;
        p.vec = true;
        return p;
    }
    // 128x128 tiles above 64 rows.  Their two-stage DMA ring (32 KiB of LDS)
    // lets four or five workgroups share a CU, and the time then follows the
    // work with no steps at whole rounds of co-resident workgroups: 5000 x
    // 4096 x 4096 1.230 ms against 1.657 in 128x256 tiles (two to a CU, 640
    // tiles: two rounds), 7168 x 4096 x 4096 1.700 against 1.944, 4096^3
    // 0.974 against 0.975 (one round of each).  128x256 stays selectable
    // (CLOVE_GEMM_CFG=5).  Where the DMA kernels take the shape, choose_tiles
    // weighs 64x128 tiles and the K split against them (either tiling runs
    // on DMA whatever the alignment of the rows).
    int cfg = M <= 32 ? CFG_32x128 : (M <= 64 ? (long_k64 ? CFG_64x128 : CFG_64x64) : CFG_128x128);
    if (force_cfg >= 0 && force_cfg < CFG_COUNT) cfg = force_cfg;
    const bool modeled = force_cfg < 0 && M > 64 && (uint64_t)M * K * 4 < (1ull << 31) &&
                         b_bytes < (1ull << 31);
    TileChoice choice{cfg, 1};
    // Both operands in the 4-byte DMA form (K and N not multiples of 4, or
    // unaligned operands) take 64x128 tiles: a 128x128 tile would issue 16
    // DMAs per wave and slab and hold 121 VGPRs (749 x 3725 x 1673: 67
    // TFLOP/s against 91 in 64x128 tiles; over the 12 such shapes timed the
    // mean time fell about 2%, the others within run-to-run noise).  With one
    // operand in that form the choice stays open (restricting it too cost
    // 1-4% on most such shapes).
    const bool both_four_byte = (K % 4 != 0 || !a_aligned) && (N % 4 != 0 || !b_aligned);
    if (modeled) choice = choose_tiles(M, N, K, num_cus, both_four_byte);
    // 33-64 rows on 64x128 tiles take the model's K split too: 40 x 2048 x
    // 40001 157 -> 104 us, 33 x 4096 x 50257 316 -> 241, 64 x 4096 x 50256
    // 280 -> 247, 64 x 1024 x 32000 45 -> 41 (40 x 4096 x 32000 149 -> 151,
    // 64 x 8192 x 8192 78 -> 82 the other way; the rest within 1%).
    const bool modeled64 = long_k64 && force_cfg < 0;
    if (modeled64) choice = choose_tiles(M, N, K, num_cus, true);
    cfg = choice.cfg;
    p.cfg = cfg;
    const int BM = kCfgBM[cfg], BN = kCfgBN[cfg], BK = kCfgBK[cfg];
    p.tiles_n = (N + BN - 1) / BN;
    p.tiles = ((M + BM - 1) / BM) * p.tiles_n;
    // Shapes choose_tiles does not take: split K when the tiles alone cannot
    // fill the chip, and for 128-row
    // tiles over K >= 1024 when they give a CU fewer than two workgroups (one
    // alone waits on its own loads and barriers: 1024 x 4096 x 4096 in 256
    // tiles ran 0.276 ms, 2047 x 4096 x 2052 in 272 0.497 ms): aim for about
    // two, each split covering at least four K slabs.
    const int slabs = (K + BK - 1) / BK;
    int splits = 1;
    if (modeled || modeled64) {
        splits = choice.splits;
    } else if (p.tiles < num_cus || (BM == 128 && slabs >= 64 && p.tiles < 2 * num_cus)) {
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

void gemm_f32_grouped(const GemmPlan *plans, const float *const *A, const float *const *B,
                      float *const *C, const GemmEpilogue *epi, int count, hipStream_t s) {
    if (count <= 0 || count > kGemmGroupMax) return;
    GroupedArgs ga{};
    int waves = 2, start = 0;
    for (int i = 0; i < count; ++i) {
        const GemmPlan &p = plans[i];
        // one 16-row block per tile in the grouped kernel
        const int tiles_n = (p.N + 15) / 16;
        const int tiles = ((p.M + 15) / 16) * tiles_n;
        ga.prob[i] = GemmArgs{A[i], B[i], C[i], nullptr, p.M, p.N, p.K, tiles_n, p.k_per_split, 1,
                              epi[i], tiles, (tiles + 7) / 8};
        ga.starts[i] = start;
        start += tiles;
        waves = std::max(waves, p.waves);
    }
    ga.starts[count] = start;
    ga.count = count;
    if (start == 0) return;
    switch (waves) {
    case 2: gemm_small_grouped_kernel<2><<<(unsigned)start, 128, 0, s>>>(ga); break;
    case 4: gemm_small_grouped_kernel<4><<<(unsigned)start, 256, 0, s>>>(ga); break;
    case 8: gemm_small_grouped_kernel<8><<<(unsigned)start, 512, 0, s>>>(ga); break;
    default: gemm_small_grouped_kernel<16><<<(unsigned)start, 1024, 0, s>>>(ga); break;
    }
}

bool gemm_f32_transposed(const GemmPlan &p, const float *A, const float *B, float *C, float *ws,
                         bool ta, bool tb, hipStream_t s) {
    if (ta == tb) return false;  // exactly one operand read transposed (the matmul backward)
    if (p.small || p.skinny || p.strip || p.K <= 0 || (p.splits > 1 && !ws)) return false;
    if (((reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B)) & 15) != 0) return false;
    if (p.cfg != CFG_128x256 && p.cfg != CFG_128x128 && p.cfg != CFG_64x128) return false;
    const GemmArgs g{A, B, C, ws, p.M, p.N, p.K, p.tiles_n, p.k_per_split, p.splits,
                     GemmEpilogue{}, p.tiles, (p.tiles + 7) / 8};
    const dim3 grid((unsigned)(g.per_xcd * 8), (unsigned)p.splits);
    // split K: each split parks its tile in ws, then the splits are summed in
    // order (gemm_f32's reduce)
    auto reduce = [&] {
        if (p.splits <= 1) return;
        const int BM = kCfgBM[p.cfg], BN = kCfgBN[p.cfg];
        const int64_t work = (int64_t)p.tiles * BM * (BN / 4);
        int64_t blocks = (work + 63) / 64;
        if (blocks > 32768) blocks = 32768;
        gemm_splitk_reduce<<<(unsigned)blocks, 64, 0, s>>>(ws, C, p.M, p.N, BM, BN, p.tiles_n,
                                                           p.tiles, p.splits, GemmEpilogue{});
    };
    if (!p.interior) {
        // ragged tiles or a K tail: the DMA kernel's edge form, whose 16-byte
        // pieces need whole quads along each stored row (A^T's M and B's N
        // for ta, K for tb); anything else transposes first
        const char *v = std::getenv("CLOVE_GEMM_DMA");
        const bool rows4 = ta ? (p.M % 4 == 0 && p.N % 4 == 0) : p.K % 4 == 0;
        if ((v && *v && std::atoi(v) == 0) || !rows4 ||
            (uint64_t)p.M * p.K * 4 >= (1ull << 31) || (uint64_t)p.K * p.N * 4 >= (1ull << 31))
            return false;
        constexpr int ST = dma_stages(128);
        if (p.cfg == CFG_128x256) {
            if (ta)
                gemm_f32_dma_kernel<128, 256, 16, 64, 128, false, true, false, kDmaStages, true>
                    <<<grid, 256, 0, s>>>(g);
            else
                gemm_f32_dma_kernel<128, 256, 16, 64, 128, false, false, true, kDmaStages, true>
                    <<<grid, 256, 0, s>>>(g);
        } else if (p.cfg == CFG_64x128) {
            if (ta)
                gemm_f32_dma_kernel<64, 128, 16, 32, 64, false, true, false, ST, true>
                    <<<grid, 256, 0, s>>>(g);
            else
                gemm_f32_dma_kernel<64, 128, 16, 32, 64, false, false, true, ST, true>
                    <<<grid, 256, 0, s>>>(g);
        } else {
            if (ta)
                gemm_f32_dma_kernel<128, 128, 16, 64, 64, false, true, false, ST, true>
                    <<<grid, 256, 0, s>>>(g);
            else
                gemm_f32_dma_kernel<128, 128, 16, 64, 64, false, false, true, ST, true>
                    <<<grid, 256, 0, s>>>(g);
        }
        reduce();
        return true;
    }
    if (p.cfg == CFG_64x128) {
        // DMA only: the register-staged kernel has no transposed 64x128 form
        if (!dma_ok(p, 64, 128)) return false;
        constexpr int ST = dma_stages(128);
        if (ta)
            gemm_f32_dma_kernel<64, 128, 16, 32, 64, false, true, false, ST><<<grid, 256, 0, s>>>(g);
        else
            gemm_f32_dma_kernel<64, 128, 16, 32, 64, false, false, true, ST><<<grid, 256, 0, s>>>(g);
        reduce();
        return true;
    }
    if (p.cfg == CFG_128x256 && dma_ok(p, 128, 256)) {
        if (ta)
            gemm_f32_dma_kernel<128, 256, 16, 64, 128, false, true, false><<<grid, 256, 0, s>>>(g);
        else
            gemm_f32_dma_kernel<128, 256, 16, 64, 128, false, false, true><<<grid, 256, 0, s>>>(g);
    } else if (p.cfg == CFG_128x128 && dma_ok(p, 128, 128)) {
        constexpr int ST = dma_stages(128);
        if (ta)
            gemm_f32_dma_kernel<128, 128, 16, 64, 64, false, true, false, ST><<<grid, 256, 0, s>>>(g);
        else
            gemm_f32_dma_kernel<128, 128, 16, 64, 64, false, false, true, ST><<<grid, 256, 0, s>>>(g);
    } else if (p.cfg == CFG_128x256) {
        if (ta)
            gemm_f32_mfma_kernel<128, 256, 16, 64, 128, false, true, false, true, false>
                <<<grid, 256, 0, s>>>(g);
        else
            gemm_f32_mfma_kernel<128, 256, 16, 64, 128, false, true, false, false, true>
                <<<grid, 256, 0, s>>>(g);
    } else {
        if (ta)
            gemm_f32_mfma_kernel<128, 128, 16, 64, 64, false, true, false, true, false>
                <<<grid, 256, 0, s>>>(g);
        else
            gemm_f32_mfma_kernel<128, 128, 16, 64, 64, false, true, false, false, true>
                <<<grid, 256, 0, s>>>(g);
    }
    reduce();
    return true;
}

void gemm_f32(const GemmPlan &p, const float *A, const float *B, float *C, float *ws,
              const GemmEpilogue &epi, hipStream_t s) {
    if (p.M <= 0 || p.N <= 0) return;
    if (p.K <= 0) {
        const uint64_t total = (uint64_t)p.M * p.N;
        const uint64_t blocks = std::min<uint64_t>((total + 255) / 256, 16384);
        gemm_k0_kernel<<<(unsigned)blocks, 256, 0, s>>>(C, p.M, p.N, epi);
        return;
    }
    GemmPlan q = p;
    if (((reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B)) & 15) != 0) {
        q.vec = false;
        q.interior = false;
    }
    GemmArgs g{A, B, C, ws, p.M, p.N, p.K, p.tiles_n, p.k_per_split, p.splits, epi,
               p.tiles, (p.tiles + 7) / 8};
    if (p.small) {
        launch_small(p, g, s);
        return;
    }
    if (p.strip) {
        launch_strip(p, g, s);
        return;
    }
    if (p.skinny) {
        const dim3 grid((unsigned)p.tiles, (unsigned)p.splits);
        launch_skinny(p, g, grid, s);
        if (p.splits > 1) {
            const int BM = 32 * p.mb, BN = 32 * p.nb;
            const int64_t work = (int64_t)p.tiles * BM * (BN / 4);
            int64_t blocks = (work + 63) / 64;
            if (blocks > 32768) blocks = 32768;
            gemm_splitk_reduce<<<(unsigned)blocks, 64, 0, s>>>(ws, C, p.M, p.N, BM, BN, p.tiles_n,
                                                               p.tiles, p.splits, epi);
        }
        return;
    }
    switch (q.cfg) {
    case CFG_32x128: launch_cfg<32, 128, 32, 32, 32>(q, g, s); break;
    case CFG_64x64: launch_cfg<64, 64, 16, 32, 32>(q, g, s); break;
    case CFG_128x128: launch_cfg<128, 128, 16, 64, 64>(q, g, s); break;
    case CFG_128x128_K32: launch_cfg<128, 128, 32, 64, 64>(q, g, s); break;
    case CFG_256x128: launch_cfg<256, 128, 16, 128, 64>(q, g, s); break;
    case CFG_64x128: launch_cfg<64, 128, 16, 32, 64>(q, g, s); break;
    default: launch_cfg<128, 256, 16, 64, 128>(q, g, s); break;
    }
    if (p.splits > 1) {
        const int BM = kCfgBM[q.cfg], BN = kCfgBN[q.cfg];
        const int64_t work = (int64_t)p.tiles * BM * (BN / 4);
        int64_t blocks = (work + 63) / 64;
        if (blocks > 32768) blocks = 32768;
        gemm_splitk_reduce<<<(unsigned)blocks, 64, 0, s>>>(ws, C, p.M, p.N, BM, BN, p.tiles_n,
                                                           p.tiles, p.splits, epi);
    }
}

}  // namespace k
}  // namespace clove
