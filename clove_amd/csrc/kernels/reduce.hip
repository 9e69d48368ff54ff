// reduce.hip -- deterministic reductions of the backward pass and the
// losses, and the transpose the matmul backward uses.
//
// Reference: the broadcast-operand gradient of add / sub (CPU backend.rs:
// 1527-1538, 1800-1810; WGSL backend.rs:596-645) and the MSE / cross-entropy
// losses (CPU backend.rs:2661-2680, 2765-2772; WGSL lazy.rs:4379-4500).  The
// WGSL versions add into one f32 through a compare-and-swap loop, so their
// result depends on the order the workgroups arrive in (and the bias one
// folds a whole workgroup into the first thread's bin).  Here every sum is
// a fixed tree: partial sums in registers, combined in LDS in a fixed order,
// then one small pass over the partials, so results repeat bit for bit.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "launch.hpp"
#include "wave.h"

namespace clove {
namespace k {

namespace {

// ---- gradient of a broadcast operand: gb[j] = sum_{i % nb == j} g[i] ------

// nb >= 64: thread per column; the grid's y dimension splits the rows
// (row r holds elements r*nb .. r*nb + nb - 1) into chunks of rows_per.
// part[chunk][j] = sum over the chunk's rows, in row order.
__global__ void __launch_bounds__(256) bcast_grad_cols_kernel(const float *__restrict__ g,
                                                              uint64_t n, uint64_t nb,
                                                              uint64_t rows_per,
                                                              float *__restrict__ part) {
    const uint64_t j = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (j >= nb) return;
    const uint64_t r0 = (uint64_t)blockIdx.y * rows_per;
    float s = 0.0f;
    uint64_t i = r0 * nb + j;
    for (uint64_t r = 0; r < rows_per && i < n; ++r, i += nb) s += g[i];
    part[(uint64_t)blockIdx.y * nb + j] = s;
}

// The same with four consecutive columns per thread and 16-byte loads
// (nb % 4 == 0, g 16-byte aligned).  A workgroup of 512 threads covers
// kColQuads column quads (512 columns) of one chunk of rows: thread
// (q, r) = (tid % kColQuads, tid / kColQuads) sums its quad over rows r,
// r + kColGroups, ... of the chunk, kColBatch loads at a time, and the
// kColGroups row groups are then added in group order through LDS (a fixed
// order: deterministic).  512 workgroups at 4096 x 4096 (chunks of 64
// rows), each reading 2 KiB of every row of its chunk, each thread's loads
// in two batches of eight; bcast_grad_final_kernel then adds the 64 chunk
// partials of each column.  With the input cycled through copies the 256 MB
// last-level cache cannot hold: 14.6 us (57% of HBM peak) for both passes,
// against 19-20 us for one launch of 32-column strips over the whole height
// (128 workgroups, too few to pull 64 MiB from HBM at full rate; 12.7 us
// only while three 64 MiB copies stayed in that cache).  A form of 256
// threads covering 1024 columns ran half as many workgroups: 55% end to end
// against 57%.
constexpr int kColThreads = 512, kColQuads = 128, kColGroups = kColThreads / kColQuads;
constexpr int kColBatch = 8;
__global__ void __launch_bounds__(kColThreads) bcast_grad_cols4_kernel(const float *__restrict__ g,
                                                                       uint64_t n, uint64_t nb,
                                                                       uint64_t rows_per,
                                                                       float *__restrict__ part) {
    __shared__ cl_f4 grp_sum[kColGroups - 1][kColQuads];
    const int ql = threadIdx.x % kColQuads, grp = threadIdx.x / kColQuads;
    const uint64_t nq = nb / 4;
    const uint64_t q = (uint64_t)blockIdx.x * kColQuads + ql;
    const bool live = q < nq;
    const uint64_t r0 = (uint64_t)blockIdx.y * rows_per;
    const uint64_t rows = (n + nb - 1) / nb;
    const uint64_t r1 = r0 + rows_per < rows ? r0 + rows_per : rows;
    const uint64_t full = n / nb;  // rows wholly inside n
    const uint64_t r_full = r1 < full ? r1 : full;
    const cl_f4 *g4 = reinterpret_cast<const cl_f4 *>(g);
    cl_f4 s = {0.f, 0.f, 0.f, 0.f};
    if (live) {
        uint64_t r = r0 + grp;
        for (; r + (uint64_t)(kColBatch - 1) * kColGroups < r_full;
             r += (uint64_t)kColBatch * kColGroups) {
            cl_f4 v[kColBatch];
#pragma unroll
            for (int u = 0; u < kColBatch; ++u)
                v[u] = __builtin_nontemporal_load(g4 + (r + (uint64_t)u * kColGroups) * nq + q);
#pragma unroll
            for (int u = 0; u < kColBatch; ++u) s += v[u];
        }
        for (; r < r1; r += kColGroups) {
            if (r < full) {
                s += __builtin_nontemporal_load(g4 + r * nq + q);
            } else {  // the last, partial row
                const uint64_t i = r * nb + 4 * q;
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if (i + c < n) s[c] += g[i + c];
            }
        }
    }
    if (grp > 0) grp_sum[grp - 1][ql] = s;
    __syncthreads();
    if (grp == 0 && live) {
#pragma unroll
        for (int k = 0; k < kColGroups - 1; ++k) s += grp_sum[k][ql];
        *reinterpret_cast<cl_f4 *>(part + (uint64_t)blockIdx.y * nb + 4 * q) = s;
    }
}

// nb < 64: T = nb * (256 / nb) threads each own one column, (base + t) % nb,
// and sum every T-th element of the workgroup's chunk (chunk starts are
// multiples of T, hence of nb); the threads of one column are then added
// in thread order.  part[chunk][j].
__global__ void __launch_bounds__(256) bcast_grad_flat_kernel(const float *__restrict__ g,
                                                              uint64_t n, int nb, int iters,
                                                              float *__restrict__ part) {
    __shared__ float acc[256];
    const int T = nb * (256 / nb);
    const int t = threadIdx.x;
    const uint64_t base = (uint64_t)blockIdx.x * T * iters;
    float s = 0.0f;
    if (t < T) {
        uint64_t i = base + t;
        for (int k = 0; k < iters && i < n; ++k, i += T) s += g[i];
    }
    acc[t] = s;
    __syncthreads();
    if (t < nb) {
        float c = 0.0f;
        for (int q = t; q < T; q += nb) c += acc[q];
        part[(uint64_t)blockIdx.x * nb + t] = c;
    }
}

// gb[j] = sign * sum over chunks of part[chunk][j].  A workgroup covers 32
// columns with 8 groups of threads; group k sums chunks [k*per, (k+1)*per)
// in order, and the 8 group sums meet in LDS and are added in group order: a
// fixed order, so the result is deterministic, with 8x the parallelism of
// one thread per column.  A group's loads go out 16 at a time before any is
// added (each load-then-add would cost a memory round trip).
__global__ void __launch_bounds__(256) bcast_grad_final_kernel(const float *__restrict__ part,
                                                               uint64_t chunks, uint64_t nb,
                                                               float sign,
                                                               float *__restrict__ gb) {
    constexpr int kBatch = 16;
    __shared__ float grp[8][32];
    const int cl = threadIdx.x & 31, k = threadIdx.x >> 5;
    const uint64_t j = (uint64_t)blockIdx.x * 32 + cl;
    const uint64_t per = (chunks + 7) / 8;
    const uint64_t c0 = (uint64_t)k * per;
    const uint64_t c1 = c0 + per < chunks ? c0 + per : chunks;
    float s = 0.0f;
    if (j < nb) {
        for (uint64_t c = c0; c < c1; c += kBatch) {
            float v[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u)
                if (c + u < c1) v[u] = part[(c + u) * nb + j];
#pragma unroll
            for (int u = 0; u < kBatch; ++u)
                if (c + u < c1) s += v[u];
        }
    }
    grp[k][cl] = s;
    __syncthreads();
    if (k == 0 && j < nb) {
        float t = grp[0][cl];
#pragma unroll
        for (int q = 1; q < 8; ++q) t += grp[q][cl];
        gb[j] = sign * t;
    }
}

// ---- scalar losses ------------------------------------------------------

// Sum of squared differences over a chunk of kSqChunk elements per
// workgroup of kSqThreads threads, combined in a fixed order: part[block].
// VEC: 16-byte loads (p and t 16-byte aligned), kSqChunk / (4 kSqThreads)
// vectors of each input per thread, all issued before any arithmetic; a
// chunk reaching past n is read element by element.  16 KiB of each input
// per 512-thread workgroup streamed fastest among the shapes measured with
// inputs the last-level cache does not hold (a 64 KiB chunk per 256 threads
// read 2-4 points of HBM peak slower).
constexpr int kSqThreads = 512;
constexpr int kSqChunk = kSqThreads * 8;
template <bool VEC>
__global__ void __launch_bounds__(kSqThreads) sq_diff_partial_kernel(const float *__restrict__ p,
                                                                    const float *__restrict__ t,
                                                                    uint64_t n,
                                                                    float *__restrict__ part) {
    constexpr int kWaves = kSqThreads / 64, kVec = kSqChunk / (4 * kSqThreads);
    __shared__ float wsum[kWaves];
    const uint64_t base = (uint64_t)blockIdx.x * kSqChunk;
    float s = 0.0f;
    if (VEC && base + kSqChunk <= n) {
        const cl_f4 *p4 = reinterpret_cast<const cl_f4 *>(p + base);
        const cl_f4 *t4 = reinterpret_cast<const cl_f4 *>(t + base);
        cl_f4 vp[kVec], vt[kVec];
#pragma unroll
        for (int k = 0; k < kVec; ++k) {
            vp[k] = __builtin_nontemporal_load(p4 + k * kSqThreads + threadIdx.x);
            vt[k] = __builtin_nontemporal_load(t4 + k * kSqThreads + threadIdx.x);
        }
        cl_f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < kVec; ++k) {
            const cl_f4 d = vp[k] - vt[k];
            acc += d * d;
        }
        s = hsum4(acc);
    } else {
        for (int k = 0; k < kSqChunk / kSqThreads; ++k) {
            const uint64_t i = base + (uint64_t)k * kSqThreads + threadIdx.x;
            if (i < n) {
                const float d = p[i] - t[i];
                s += d * d;
            }
        }
    }
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        float r = wsum[0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) r += wsum[w];
        part[blockIdx.x] = r;
    }
}

// out[0] = (sign * sum of x[0..n)) / div, one workgroup, fixed order.
// Thread t sums x[t], x[t + 1024], ... in order; the 16 wave sums are added
// in wave order.  A single workgroup has nothing else to hide its load
// latency behind, so each thread's loads go out eight at a time before any
// is added: up to 8192 values cost one memory round trip.
constexpr int kSumThreads = 1024;
__global__ void __launch_bounds__(kSumThreads) ordered_sum_kernel(const float *__restrict__ x,
                                                                  uint64_t n, float sign,
                                                                  float div,
                                                                  float *__restrict__ out) {
    constexpr int kBatch = 8, kWaves = kSumThreads / 64;
    __shared__ float wsum[kWaves];
    float s = 0.0f;
    for (uint64_t base = threadIdx.x; base < n; base += (uint64_t)kBatch * kSumThreads) {
        float v[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const uint64_t i = base + (uint64_t)u * kSumThreads;
            if (i < n) v[u] = x[i];
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
            if (base + (uint64_t)u * kSumThreads < n) s += v[u];
    }
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = wsum[0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) t += wsum[w];
        out[0] = (sign * t) / div;
    }
}

// x / y correctly rounded, for a y shared by many x, from r = 1 / y (IEEE):
// q0 = x r, then one FMA correction of the remainder (Markstein's method).
// With r the correctly rounded reciprocal this is the IEEE quotient; checked
// against x / y for every integer y up to 70000 over 2000 random x each
// (normal range, both signs).  An infinite q0 (x infinite) is returned as is.
__device__ __forceinline__ float div_exact(float x, float y, float r) {
    const float q0 = x * r;
    const float q1 = __builtin_fmaf(__builtin_fmaf(-q0, y, x), r, q0);
    return __builtin_isfinite(q0) ? q1 : q0;
}

// MSE backward (backend.rs:2780-2790): grad = 2 * (p - t) * g / n, each
// step rounded in that order.  VEC: 16-byte streaming loads and stores over
// the whole vectors (p, t, grad 16-byte aligned), the tail element by element.
constexpr int kMseBwThreads = 512;
template <bool VEC>
__global__ void __launch_bounds__(kMseBwThreads) mse_backward_kernel(const float *__restrict__ p,
                                                           const float *__restrict__ t,
                                                           uint64_t n,
                                                           const float *__restrict__ grad_loss,
                                                           float *__restrict__ grad) {
    const float g = grad_loss[0];
    const float nf = (float)n;
    const float rn = 1.0f / nf;
    const uint64_t stride = (uint64_t)gridDim.x * kMseBwThreads;
    uint64_t tail = 0;
    if (VEC) {
        const uint64_t nv = n / 4;
        const cl_f4 *p4 = reinterpret_cast<const cl_f4 *>(p);
        const cl_f4 *t4 = reinterpret_cast<const cl_f4 *>(t);
        cl_f4 *g4 = reinterpret_cast<cl_f4 *>(grad);
        for (uint64_t i = (uint64_t)blockIdx.x * kMseBwThreads + threadIdx.x; i < nv;
             i += stride) {
            const cl_f4 d = __builtin_nontemporal_load(p4 + i) - __builtin_nontemporal_load(t4 + i);
            const cl_f4 x = 2.0f * d * g;
            __builtin_nontemporal_store((cl_f4){div_exact(x.x, nf, rn), div_exact(x.y, nf, rn),
                                                div_exact(x.z, nf, rn), div_exact(x.w, nf, rn)},
                                        g4 + i);
        }
        tail = 4 * nv;
    }
    for (uint64_t i = tail + (uint64_t)blockIdx.x * kMseBwThreads + threadIdx.x; i < n;
         i += stride)
        grad[i] = div_exact(2.0f * (p[i] - t[i]) * g, nf, rn);
}

// ---- transpose: out[c][r] = in[r][c] for an R x C matrix ------------------
// 64x64 tiles through LDS (pitch 65 against bank conflicts); 256 threads,
// each moving 16 elements.  Edge tiles are bounds-checked.
__global__ void __launch_bounds__(256) transpose_kernel(const float *__restrict__ in,
                                                        float *__restrict__ out, int R, int C) {
    __shared__ float tile[64][65];
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;  // 64 x 4
    const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const int r = r0 + ty + 4 * k, c = c0 + tx;
        if (r < R && c < C) tile[ty + 4 * k][tx] = in[(size_t)r * C + c];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const int c = c0 + ty + 4 * k, r = r0 + tx;
        if (r < R && c < C) out[(size_t)c * R + r] = tile[tx][ty + 4 * k];
    }
}

// Rows per chunk of the column kernel: 64, or more when that would need
// more than 16384 chunks (the grid's y dimension).  At 4096 x 4096 that is
// 512 workgroups, two per CU, each thread streaming 16 rows; 64 against 32
// rows per chunk measured 13.9 against 14.5 us there (half the partial
// rows for the final kernel to read) and 45.5 against 48.7 us at 16384 rows;
// 128 rows measured 14.3 and 48.1 us.
size_t cols_rows_per(size_t rows) {
    if (rows <= 64) return rows ? rows : 1;
    const size_t need = (rows + 16383) / 16384;
    return need > 64 ? need : 64;
}

}  // namespace

size_t broadcast_grad_workspace(size_t n, size_t nb) {
    if (nb == 0 || n == 0) return 0;
    if (nb >= 64) {
        const size_t rows = (n + nb - 1) / nb;
        const size_t rows_per = cols_rows_per(rows);
        return ((rows + rows_per - 1) / rows_per) * nb;
    }
    const size_t T = nb * (256 / nb), per = T * 64;
    return ((n + per - 1) / per) * nb;
}

void broadcast_grad(const float *g, size_t n, size_t nb, bool negate, float *part, float *gb,
                    hipStream_t s) {
    if (nb == 0) return;
    size_t chunks;
    if (nb >= 64) {
        const size_t rows = (n + nb - 1) / nb;
        const size_t rows_per = cols_rows_per(rows);
        chunks = (rows + rows_per - 1) / rows_per;
        if (chunks && nb % 4 == 0 && (reinterpret_cast<uintptr_t>(g) & 15) == 0) {
            const dim3 grid((unsigned)((nb / 4 + kColQuads - 1) / kColQuads), (unsigned)chunks);
            bcast_grad_cols4_kernel<<<grid, kColThreads, 0, s>>>(g, n, nb, rows_per, part);
        } else if (chunks) {
            const dim3 grid((unsigned)((nb + 255) / 256), (unsigned)chunks);
            bcast_grad_cols_kernel<<<grid, 256, 0, s>>>(g, n, nb, rows_per, part);
        }
    } else {
        const size_t T = nb * (256 / nb), per = T * 64;
        chunks = (n + per - 1) / per;
        if (chunks) bcast_grad_flat_kernel<<<(unsigned)chunks, 256, 0, s>>>(g, n, (int)nb, 64, part);
    }
    bcast_grad_final_kernel<<<(unsigned)((nb + 31) / 32), 256, 0, s>>>(
        part, chunks, nb, negate ? -1.0f : 1.0f, gb);
}

size_t sq_diff_workspace(size_t n) { return (n + kSqChunk - 1) / kSqChunk; }

void mse_loss(const float *p, const float *t, size_t n, float *part, float *out, hipStream_t s) {
    const size_t blocks = sq_diff_workspace(n);
    const bool vec = ((reinterpret_cast<uintptr_t>(p) | reinterpret_cast<uintptr_t>(t)) & 15) == 0;
    if (blocks && vec)
        sq_diff_partial_kernel<true><<<(unsigned)blocks, kSqThreads, 0, s>>>(p, t, n, part);
    else if (blocks)
        sq_diff_partial_kernel<false><<<(unsigned)blocks, kSqThreads, 0, s>>>(p, t, n, part);
    ordered_sum_kernel<<<1, kSumThreads, 0, s>>>(part, blocks, 1.0f, (float)n, out);
}

void ordered_sum(const float *x, size_t n, float sign, float div, float *out, hipStream_t s) {
    ordered_sum_kernel<<<1, kSumThreads, 0, s>>>(x, n, sign, div, out);
}

void mse_backward(const float *p, const float *t, size_t n, const float *grad_loss, float *grad,
                  hipStream_t s) {
    if (!n) return;
    const bool vec = ((reinterpret_cast<uintptr_t>(p) | reinterpret_cast<uintptr_t>(t) |
                       reinterpret_cast<uintptr_t>(grad)) & 15) == 0;
    // one vector per thread per pass, 512-thread workgroups (the fused
    // chains' shape), a grid of up to 8192 workgroups
    size_t blocks = ((vec ? n / 4 : n) + kMseBwThreads - 1) / kMseBwThreads;
    if (blocks > 8192) blocks = 8192;
    if (blocks == 0) blocks = 1;
    if (vec)
        mse_backward_kernel<true><<<(unsigned)blocks, kMseBwThreads, 0, s>>>(p, t, n, grad_loss, grad);
    else
        mse_backward_kernel<false><<<(unsigned)blocks, kMseBwThreads, 0, s>>>(p, t, n, grad_loss, grad);
}

void transpose(const float *in, float *out, size_t R, size_t C, hipStream_t s) {
    if (!R || !C) return;
    const dim3 grid((unsigned)((C + 63) / 64), (unsigned)((R + 63) / 64));
    transpose_kernel<<<grid, 256, 0, s>>>(in, out, (int)R, (int)C);
}

}  // namespace k
}  // namespace clove
