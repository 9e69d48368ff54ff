// rowwise.hip -- row softmax and row layer norm, and the row kernels of the
// backward pass (softmax backward, cross entropy and its backward).
//
// Reference: the CPU kernels (softmax backend.rs:2102-2125, layer_norm
// backend.rs:2380-2405) and the lazy WGSL (lazy.rs:4718-4737, 4786-4806),
// which runs ONE THREAD PER ROW and reads each row three times with a 16 KiB
// stride between neighbouring threads.
//
// Here a whole wavefront owns a row: lanes read 16-byte vectors so a wave
// instruction covers 1 KiB of contiguous row, the row stays in VGPRs between
// the passes (so HBM sees exactly one read and one write per element), and
// the max / sum / mean / variance reductions are wave64 butterflies with no
// LDS and no barriers.  Rows wider than 1024 columns (all but layer norm)
// take a whole workgroup of 512 threads instead, which streams faster; see
// the row-per-workgroup section below.
//
// Per-element arithmetic is kept to a few VALU operations so the kernels stay
// bound by HBM: exp(x) is the hardware 2^x (v_exp_f32) of x*log2(e) (relative
// error ~6e-8 |x|, about 1e-6 over the softmax range), and the per-row
// division by the sum (softmax) or by the standard deviation (layer norm) is
// one IEEE reciprocal per row times a multiply per element (<= 1.5 ulp).
// The CPU kernels divide per element; both stay far inside the 1e-4 parity
// bound.  Rows whose width is not a multiple of 4, or wider
// than 8192, go through a looped wave-per-row kernel that re-reads the row.
#include <hip/hip_runtime.h>

#include <cmath>

#include "launch.hpp"
#include "wave.h"

namespace clove {
namespace k {

namespace {

constexpr int kRowsPerBlock = 4;  // one row per wave, 4 waves per block

__device__ __forceinline__ float fast_exp(float x) {
    return __builtin_amdgcn_exp2f(x * 1.44269504088896341f);
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

template <int VPT>
__global__ void __launch_bounds__(256) softmax_wave_kernel(const float *__restrict__ x,
                                                           float *__restrict__ y, int rows,
                                                           int cols) {
    const int lane = threadIdx.x & 63;
    const long row = (long)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int nvec = cols >> 2;
    const cl_f4 *xr = reinterpret_cast<const cl_f4 *>(x + row * (long)cols);
    cl_f4 *yr = reinterpret_cast<cl_f4 *>(y + row * (long)cols);
    cl_f4 v[VPT];
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int c = lane + 64 * i;
        v[i] = c < nvec ? __builtin_nontemporal_load(xr + c)
                        : (cl_f4){-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    }
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < VPT; ++i) m = fmaxf(m, hmax4(v[i]));
    m = wave_max(m);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        if (lane + 64 * i < nvec) {
            v[i] = (cl_f4){fast_exp(v[i].x - m), fast_exp(v[i].y - m), fast_exp(v[i].z - m),
                           fast_exp(v[i].w - m)};
            s += hsum4(v[i]);
        }
    }
    const float inv = 1.0f / wave_sum(s);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int c = lane + 64 * i;
        if (c < nvec) __builtin_nontemporal_store(v[i] * inv, yr + c);
    }
}

// gamma and beta are staged in LDS once per workgroup (2 * cols floats):
// every row of the workgroup reads them, and fetching them from L2 per row
// costs as much traffic as the rows themselves (at 4096 columns the pair is
// 32 KiB, the size of the vector L1).  The row's own loads are issued first
// so the staging overlaps them.
template <int VPT>
__global__ void __launch_bounds__(256) layer_norm_wave_kernel(const float *__restrict__ x,
                                                              const float *__restrict__ gamma,
                                                              const float *__restrict__ beta,
                                                              float *__restrict__ y, int rows,
                                                              int cols, float eps) {
    extern __shared__ cl_f4 s_gb[];  // [nvec] gamma, then [nvec] beta
    const int lane = threadIdx.x & 63;
    const long row = (long)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    const bool live = row < rows;
    const int nvec = cols >> 2;
    const cl_f4 *xr = reinterpret_cast<const cl_f4 *>(x + (live ? row : 0) * (long)cols);
    cl_f4 v[VPT];
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int c = lane + 64 * i;
        v[i] = (live && c < nvec) ? __builtin_nontemporal_load(xr + c) : (cl_f4){0.f, 0.f, 0.f, 0.f};
    }
    const cl_f4 *g4 = reinterpret_cast<const cl_f4 *>(gamma);
    const cl_f4 *b4 = reinterpret_cast<const cl_f4 *>(beta);
    for (int c = threadIdx.x; c < nvec; c += 256) {
        s_gb[c] = g4[c];
        s_gb[nvec + c] = b4[c];
    }
    __syncthreads();
    if (!live) return;
    cl_f4 *yr = reinterpret_cast<cl_f4 *>(y + row * (long)cols);
#pragma unroll
    for (int i = 0; i < VPT; ++i) s += hsum4(v[i]);
    const float n = (float)cols;
    const float mean = wave_sum(s) / n;
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        if (lane + 64 * i < nvec) {
            const cl_f4 d = v[i] - mean;
            q += hsum4(d * d);
        }
    }
    const float var = wave_sum(q) / n;
    const float rsd = 1.0f / sqrtf(var + eps);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int c = lane + 64 * i;
        if (c < nvec) {
            const cl_f4 o = ((v[i] - mean) * rsd) * s_gb[c] + s_gb[nvec + c];
            __builtin_nontemporal_store(o, yr + c);
        }
    }
}

// Any width: one wave per row, the row re-read from memory on each pass.
__global__ void __launch_bounds__(256) softmax_loop_kernel(const float *__restrict__ x,
                                                           float *__restrict__ y, int rows,
                                                           int cols) {
    const int lane = threadIdx.x & 63;
    const long row = (long)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *xr = x + row * (long)cols;
    float *yr = y + row * (long)cols;
    // pass 1: running (max, sum of exp) per lane, then merged across lanes
    float m = -INFINITY, s = 0.0f;
    for (int c = lane; c < cols; c += 64) {
        const float xv = xr[c];
        const float nm = fmaxf(m, xv);
        s = (m == -INFINITY ? 0.0f : s * expf(m - nm)) + expf(xv - nm);
        m = nm;
    }
    const float gm = wave_max(m);
    s = (m == -INFINITY) ? 0.0f : s * expf(m - gm);
    s = wave_sum(s);
    for (int c = lane; c < cols; c += 64) yr[c] = expf(xr[c] - gm) / s;
}

__global__ void __launch_bounds__(256) layer_norm_loop_kernel(const float *__restrict__ x,
                                                              const float *__restrict__ gamma,
                                                              const float *__restrict__ beta,
                                                              float *__restrict__ y, int rows,
                                                              int cols, float eps) {
    const int lane = threadIdx.x & 63;
    const long row = (long)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *xr = x + row * (long)cols;
    float *yr = y + row * (long)cols;
    const float n = (float)cols;
    float s = 0.0f;
    for (int c = lane; c < cols; c += 64) s += xr[c];
    const float mean = wave_sum(s) / n;
    float q = 0.0f;
    for (int c = lane; c < cols; c += 64) {
        const float d = xr[c] - mean;
        q += d * d;
    }
    const float sd = sqrtf(wave_sum(q) / n + eps);
    for (int c = lane; c < cols; c += 64) yr[c] = ((xr[c] - mean) / sd) * gamma[c] + beta[c];
}

// ---- backward and loss rows ----------------------------------------------

// Softmax backward (backend.rs:2163-2183): dx = y * (dy - sum(dy * y)) per
// row, the row of y and of dy held in registers.
template <int VPT>
__global__ void __launch_bounds__(256) softmax_bw_wave_kernel(const float *__restrict__ y,
                                                              const float *__restrict__ dy,
                                                              float *__restrict__ dx, int rows,
                                                              int cols) {
    const int lane = threadIdx.x & 63;
    const long row = (long)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int nvec = cols >> 2;
    const cl_f4 *yr = reinterpret_cast<const cl_f4 *>(y + row * (long)cols);
    const cl_f4 *gr = reinterpret_cast<const cl_f4 *>(dy + row * (long)cols);
    cl_f4 *o = reinterpret_cast<cl_f4 *>(dx + row * (long)cols);
    cl_f4 vy[VPT], vg[VPT];
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int c = lane + 64 * i;
        const bool in = c < nvec;
        vy[i] = in ? __builtin_nontemporal_load(yr + c) : (cl_f4){0.f, 0.f, 0.f, 0.f};
        vg[i] = in ? __builtin_nontemporal_load(gr + c) : (cl_f4){0.f, 0.f, 0.f, 0.f};
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) s += hsum4(vg[i] * vy[i]);
    s = wave_sum(s);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int c = lane + 64 * i;
        if (c < nvec) __builtin_nontemporal_store(vy[i] * (vg[i] - s), o + c);
    }
}

__global__ void __launch_bounds__(256) softmax_bw_loop_kernel(const float *__restrict__ y,
                                                              const float *__restrict__ dy,
                                                              float *__restrict__ dx, int rows,
                                                              int cols) {
    const int lane = threadIdx.x & 63;
    const long row = (long)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *yr = y + row * (long)cols, *gr = dy + row * (long)cols;
    float *o = dx + row * (long)cols;
    float s = 0.0f;
    for (int c = lane; c < cols; c += 64) s += gr[c] * yr[c];
    s = wave_sum(s);
    for (int c = lane; c < cols; c += 64) o[c] = yr[c] * (gr[c] - s);
}

// Rust's `f32 as usize` saturates: NaN and negative targets read class 0.
__device__ __forceinline__ long target_class(float v) {
    if (!(v > 0.0f)) return 0;
    return v >= 9.0e18f ? (long)9.0e18 : (long)v;
}

// Cross entropy, one wave per row (backend.rs:2661-2680): row value
// v = (l[t] - max) - ln(sum exp(l - max)); the loss is -sum(v) / rows, which
// ordered_sum (reduce.hip) adds in a fixed order.  Rows at or past `used` (no target)
// give 0; a class >= cols raises the error flag and gives 0.
// MODE 0 writes v to rowv[row].  MODE 1 is the backward (backend.rs:
// 2686-2712): grad = (exp(l - max) / sum - [j == t]) * g / rows.
template <int VPT, int MODE>
__global__ void __launch_bounds__(256) cross_entropy_wave_kernel(
    const float *__restrict__ logits, const float *__restrict__ targets, long used, int rows,
    int cols, const float *__restrict__ grad_loss, float *__restrict__ out, int *err_flag) {
    const int lane = threadIdx.x & 63;
    const long row = (long)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int nvec = cols >> 2;
    cl_f4 *go = MODE == 1 ? reinterpret_cast<cl_f4 *>(out + row * (long)cols) : nullptr;
    // The row's loads go out first: read after the target (and a branch on
    // it), they would wait one memory latency per row.
    const cl_f4 *lr = reinterpret_cast<const cl_f4 *>(logits + row * (long)cols);
    cl_f4 v[VPT];
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int c = lane + 64 * i;
        v[i] = c < nvec ? __builtin_nontemporal_load(lr + c)
                        : (cl_f4){-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    }
    long t = -1;
    if (row < used) {
        t = target_class(targets[row]);
        if (t >= cols) {
            if (lane == 0) atomicOr(err_flag, kErrClassRange);
            t = -1;
        }
    }
    if (t < 0) {  // no target (or a bad one): the row contributes nothing
        if (MODE == 0) {
            if (lane == 0) out[row] = 0.0f;
        } else {
            for (int c = lane; c < nvec; c += 64) go[c] = (cl_f4){0.f, 0.f, 0.f, 0.f};
        }
        return;
    }
    // l[t] from the registers of the lane that holds it (vector t/4 lives in
    // lane (t/4) % 64, slot (t/4) / 64), not from a second global load.
    float lt = 0.0f;
    if (MODE == 0) {
        const int tv = (int)(t >> 2), ts = (int)(t & 3);
#pragma unroll
        for (int i = 0; i < VPT; ++i)
            if (lane + 64 * i == tv) lt = v[i][ts];
        lt = __shfl(lt, tv & 63, 64);
    }
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < VPT; ++i) m = fmaxf(m, hmax4(v[i]));
    m = wave_max(m);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        if (lane + 64 * i < nvec) {
            v[i] = (cl_f4){fast_exp(v[i].x - m), fast_exp(v[i].y - m), fast_exp(v[i].z - m),
                           fast_exp(v[i].w - m)};
            s += hsum4(v[i]);
        }
    }
    s = wave_sum(s);
    if (MODE == 0) {
        if (lane == 0) out[row] = (lt - m) - logf(s);
        return;
    }
    const float inv = 1.0f / s;
    const float g = grad_loss[0];
    const float fr = (float)rows;
    const float rr = 1.0f / fr;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int c = lane + 64 * i;
        if (c < nvec) {
            cl_f4 p = v[i] * inv;
            const long j0 = 4l * c;
            if (t >= j0 && t < j0 + 4) p[t - j0] -= 1.0f;
            const cl_f4 x = p * g;
            __builtin_nontemporal_store((cl_f4){div_exact(x.x, fr, rr), div_exact(x.y, fr, rr),
                                                div_exact(x.z, fr, rr), div_exact(x.w, fr, rr)},
                                        go + c);
        }
    }
}

// Any width: the same, re-reading the row.
template <int MODE>
__global__ void __launch_bounds__(256) cross_entropy_loop_kernel(
    const float *__restrict__ logits, const float *__restrict__ targets, long used, int rows,
    int cols, const float *__restrict__ grad_loss, float *__restrict__ out, int *err_flag) {
    const int lane = threadIdx.x & 63;
    const long row = (long)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    float *go = MODE == 1 ? out + row * (long)cols : nullptr;
    long t = -1;
    if (row < used) {
        t = target_class(targets[row]);
        if (t >= cols) {
            if (lane == 0) atomicOr(err_flag, kErrClassRange);
            t = -1;
        }
    }
    if (t < 0) {
        if (MODE == 0) {
            if (lane == 0) out[row] = 0.0f;
        } else {
            for (int c = lane; c < cols; c += 64) go[c] = 0.0f;
        }
        return;
    }
    const float *lr = logits + row * (long)cols;
    float m = -INFINITY;
    for (int c = lane; c < cols; c += 64) m = fmaxf(m, lr[c]);
    m = wave_max(m);
    float s = 0.0f;
    for (int c = lane; c < cols; c += 64) s += fast_exp(lr[c] - m);
    s = wave_sum(s);
    if (MODE == 0) {
        if (lane == 0) out[row] = (lr[t] - m) - logf(s);
        return;
    }
    const float inv = 1.0f / s, g = grad_loss[0], fr = (float)rows;
    for (int c = lane; c < cols; c += 64) {
        const float p = fast_exp(lr[c] - m) * inv - (c == t ? 1.0f : 0.0f);
        go[c] = (p * g) / fr;
    }
}

// ---- one row per workgroup -------------------------------------------------
//
// Rows wider than 1024 columns take a whole workgroup of kBlockThreads
// threads per row, P 16-byte vectors per thread (vector c of the row lives in
// thread c % kBlockThreads, slot c / kBlockThreads).  Measured on MI355X
// with inputs cycled so the last-level cache holds none of them, a
// [8192, 4096] softmax ran at 78.9% of HBM peak this way against 69.9% with
// one wave per row (256 threads: 76.0%), and a plain 128 MiB read at 82.4%
// against 76.3%: one 16 KiB row read by eight waves at once instead of four
// rows by four waves.  The row's reductions are wave butterflies, then the
// eight wave results added (or maxed) in wave order through LDS, so results
// stay deterministic.  Per element the arithmetic is the wave kernels'.
// Layer norm keeps one wave per row: with a row per workgroup every row
// reads gamma and beta (twice the row's bytes) from the L2, and it measured
// 65-71% (one to four rows per workgroup, all loaded at once) and 63-69%
// (4-16 rows walked in order, gamma and beta in registers, the next row
// prefetched) against the wave kernel's 75%, which stages them in LDS once
// per four rows.
constexpr int kBlockThreads = 512;
constexpr int kBlockWaves = kBlockThreads / 64;

// Workgroup-wide max / sum; every thread gets the result.  Each call needs
// its own `slot` (kBlockWaves floats of LDS): a slot reused by a later
// reduction could be overwritten while a slow wave still reads it.
__device__ __forceinline__ float block_max(float v, float *slot) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) slot[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = slot[0];
#pragma unroll
    for (int w = 1; w < kBlockWaves; ++w) r = fmaxf(r, slot[w]);
    return r;
}

__device__ __forceinline__ float block_sum(float v, float *slot) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) slot[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = slot[0];
#pragma unroll
    for (int w = 1; w < kBlockWaves; ++w) r += slot[w];
    return r;
}

template <int P>
__global__ void __launch_bounds__(kBlockThreads) softmax_block_kernel(const float *__restrict__ x,
                                                                      float *__restrict__ y,
                                                                      int cols) {
    __shared__ float red[2][kBlockWaves];
    const long row = blockIdx.x;
    const int nvec = cols >> 2;
    const cl_f4 *xr = reinterpret_cast<const cl_f4 *>(x + row * (long)cols);
    cl_f4 *yr = reinterpret_cast<cl_f4 *>(y + row * (long)cols);
    cl_f4 v[P];
#pragma unroll
    for (int i = 0; i < P; ++i) {
        const int c = threadIdx.x + kBlockThreads * i;
        v[i] = c < nvec ? __builtin_nontemporal_load(xr + c)
                        : (cl_f4){-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    }
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < P; ++i) m = fmaxf(m, hmax4(v[i]));
    m = block_max(m, red[0]);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < P; ++i) {
        if (threadIdx.x + kBlockThreads * i < nvec) {
            v[i] = (cl_f4){fast_exp(v[i].x - m), fast_exp(v[i].y - m), fast_exp(v[i].z - m),
                           fast_exp(v[i].w - m)};
            s += hsum4(v[i]);
        }
    }
    const float inv = 1.0f / block_sum(s, red[1]);
#pragma unroll
    for (int i = 0; i < P; ++i) {
        const int c = threadIdx.x + kBlockThreads * i;
        if (c < nvec) __builtin_nontemporal_store(v[i] * inv, yr + c);
    }
}

template <int P>
__global__ void __launch_bounds__(kBlockThreads) softmax_bw_block_kernel(
    const float *__restrict__ y, const float *__restrict__ dy, float *__restrict__ dx, int cols) {
    __shared__ float red[kBlockWaves];
    const long row = blockIdx.x;
    const int nvec = cols >> 2;
    const cl_f4 *yr = reinterpret_cast<const cl_f4 *>(y + row * (long)cols);
    const cl_f4 *gr = reinterpret_cast<const cl_f4 *>(dy + row * (long)cols);
    cl_f4 *o = reinterpret_cast<cl_f4 *>(dx + row * (long)cols);
    cl_f4 vy[P], vg[P];
#pragma unroll
    for (int i = 0; i < P; ++i) {
        const int c = threadIdx.x + kBlockThreads * i;
        const bool in = c < nvec;
        vy[i] = in ? __builtin_nontemporal_load(yr + c) : (cl_f4){0.f, 0.f, 0.f, 0.f};
        vg[i] = in ? __builtin_nontemporal_load(gr + c) : (cl_f4){0.f, 0.f, 0.f, 0.f};
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < P; ++i) s += hsum4(vg[i] * vy[i]);
    s = block_sum(s, red);
#pragma unroll
    for (int i = 0; i < P; ++i) {
        const int c = threadIdx.x + kBlockThreads * i;
        if (c < nvec) __builtin_nontemporal_store(vy[i] * (vg[i] - s), o + c);
    }
}

// Cross entropy and its backward with a workgroup per row (the wave
// kernel's contract and arithmetic).  l[target] comes from the registers of
// the thread holding it, through LDS, published before the max reduction's
// barrier.
template <int P, int MODE>
__global__ void __launch_bounds__(kBlockThreads) cross_entropy_block_kernel(
    const float *__restrict__ logits, const float *__restrict__ targets, long used, int rows,
    int cols, const float *__restrict__ grad_loss, float *__restrict__ out, int *err_flag) {
    __shared__ float red[2][kBlockWaves];
    __shared__ float s_lt;
    const long row = blockIdx.x;
    const int nvec = cols >> 2;
    const cl_f4 *lr = reinterpret_cast<const cl_f4 *>(logits + row * (long)cols);
    cl_f4 *go = MODE == 1 ? reinterpret_cast<cl_f4 *>(out + row * (long)cols) : nullptr;
    cl_f4 v[P];
#pragma unroll
    for (int i = 0; i < P; ++i) {
        const int c = threadIdx.x + kBlockThreads * i;
        v[i] = c < nvec ? __builtin_nontemporal_load(lr + c)
                        : (cl_f4){-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    }
    long t = -1;  // the same for every thread of the row
    if (row < used) {
        t = target_class(targets[row]);
        if (t >= cols) {
            if (threadIdx.x == 0) atomicOr(err_flag, kErrClassRange);
            t = -1;
        }
    }
    if (t < 0) {
        if (MODE == 0) {
            if (threadIdx.x == 0) out[row] = 0.0f;
        } else {
            for (int c = threadIdx.x; c < nvec; c += kBlockThreads)
                go[c] = (cl_f4){0.f, 0.f, 0.f, 0.f};
        }
        return;
    }
    if (MODE == 0) {
        const int tv = (int)(t >> 2), ts = (int)(t & 3);
        if (tv % kBlockThreads == (int)threadIdx.x) {
#pragma unroll
            for (int i = 0; i < P; ++i)
                if (i == tv / kBlockThreads) s_lt = v[i][ts];
        }
    }
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < P; ++i) m = fmaxf(m, hmax4(v[i]));
    m = block_max(m, red[0]);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < P; ++i) {
        if (threadIdx.x + kBlockThreads * i < nvec) {
            v[i] = (cl_f4){fast_exp(v[i].x - m), fast_exp(v[i].y - m), fast_exp(v[i].z - m),
                           fast_exp(v[i].w - m)};
            s += hsum4(v[i]);
        }
    }
    s = block_sum(s, red[1]);
    if (MODE == 0) {
        if (threadIdx.x == 0) out[row] = (s_lt - m) - logf(s);
        return;
    }
    const float inv = 1.0f / s;
    const float g = grad_loss[0];
    const float fr = (float)rows;
    const float rr = 1.0f / fr;
#pragma unroll
    for (int i = 0; i < P; ++i) {
        const int c = threadIdx.x + kBlockThreads * i;
        if (c < nvec) {
            cl_f4 p = v[i] * inv;
            const long j0 = 4l * c;
            if (t >= j0 && t < j0 + 4) p[t - j0] -= 1.0f;
            const cl_f4 xg = p * g;
            __builtin_nontemporal_store((cl_f4){div_exact(xg.x, fr, rr), div_exact(xg.y, fr, rr),
                                                div_exact(xg.z, fr, rr), div_exact(xg.w, fr, rr)},
                                        go + c);
        }
    }
}

// Cross entropy forward with two rows per workgroup (the block kernel's
// per-row arithmetic and reduction order, so the same bits): each thread
// holds P vectors of both rows, and the two rows' maxima and sums go through
// the same butterflies and the same two barriers.  Measured at [8192, 4096]
// with cold inputs: 21.3-21.4 us against 22.0-24.0 us for one row per
// workgroup (four rows: 23.2 us): twice the bytes in flight per workgroup at
// the same barrier count.  A row past `rows` (odd row counts) loads nothing
// and writes nothing.
template <int P>
__global__ void __launch_bounds__(kBlockThreads) cross_entropy_rows2_kernel(
    const float *__restrict__ logits, const float *__restrict__ targets, long used, int rows,
    int cols, float *__restrict__ out, int *err_flag) {
    __shared__ float red[2][2][kBlockWaves];
    __shared__ float s_lt[2];
    const long row0 = 2L * blockIdx.x;
    const int nvec = cols >> 2;
    cl_f4 v[2][P];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const bool live = row0 + r < rows;
        const cl_f4 *lr = reinterpret_cast<const cl_f4 *>(logits + (row0 + r) * (long)cols);
#pragma unroll
        for (int i = 0; i < P; ++i) {
            const int c = threadIdx.x + kBlockThreads * i;
            v[r][i] = (live && c < nvec) ? __builtin_nontemporal_load(lr + c)
                                         : (cl_f4){-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        }
    }
    long t[2];  // the same for every thread of the row; -1: the row counts 0
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const long row = row0 + r;
        t[r] = -1;
        if (row < used && row < rows) {
            t[r] = target_class(targets[row]);
            if (t[r] >= cols) {
                if (threadIdx.x == 0) atomicOr(err_flag, kErrClassRange);
                t[r] = -1;
            }
        }
        if (t[r] >= 0) {
            const int tv = (int)(t[r] >> 2), ts = (int)(t[r] & 3);
            if (tv % kBlockThreads == (int)threadIdx.x) {
#pragma unroll
                for (int i = 0; i < P; ++i)
                    if (i == tv / kBlockThreads) s_lt[r] = v[r][i][ts];
            }
        }
    }
    float m[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        m[r] = -INFINITY;
#pragma unroll
        for (int i = 0; i < P; ++i) m[r] = fmaxf(m[r], hmax4(v[r][i]));
        m[r] = wave_max(m[r]);
        if ((threadIdx.x & 63) == 0) red[0][r][threadIdx.x >> 6] = m[r];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        float x = red[0][r][0];
#pragma unroll
        for (int w = 1; w < kBlockWaves; ++w) x = fmaxf(x, red[0][r][w]);
        m[r] = x;
    }
    float sm[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        sm[r] = 0.0f;
#pragma unroll
        for (int i = 0; i < P; ++i) {
            if (threadIdx.x + kBlockThreads * i < nvec) {
                const cl_f4 e = {fast_exp(v[r][i].x - m[r]), fast_exp(v[r][i].y - m[r]),
                                 fast_exp(v[r][i].z - m[r]), fast_exp(v[r][i].w - m[r])};
                sm[r] += hsum4(e);
            }
        }
        sm[r] = wave_sum(sm[r]);
        if ((threadIdx.x & 63) == 0) red[1][r][threadIdx.x >> 6] = sm[r];
    }
    __syncthreads();
    if (threadIdx.x < 2) {
        const int r = threadIdx.x;
        const long row = row0 + r;
        if (row < rows) {
            float x = red[1][r][0];
#pragma unroll
            for (int w = 1; w < kBlockWaves; ++w) x += red[1][r][w];
            out[row] = t[r] < 0 ? 0.0f : (s_lt[r] - m[r]) - logf(x);
        }
    }
}

// Vectors per thread of the row-per-workgroup kernels for this width, or 0
// for the one-wave-per-row kernels (width not a multiple of 4, at most 1024
// columns, or beyond 16 vectors per thread).
int pick_block_p(int cols) {
    if (cols % 4 != 0) return 0;
    const int nvec = cols / 4;
    if (nvec <= 256) return 0;
    int p = 1;
    while (p * kBlockThreads < nvec) p <<= 1;
    return p <= 16 ? p : 0;
}

int pick_vpt(int cols) {
    if (cols % 4 != 0) return 0;
    const int need = (cols / 4 + 63) / 64;
    int v = 1;
    while (v < need) v <<= 1;
    return v <= 32 ? v : 0;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

void softmax_rows(const float *x, float *y, size_t rows, size_t cols, hipStream_t s) {
    if (!rows || !cols) return;
    const unsigned grid = (unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock);
    const int r = (int)rows, c = (int)cols;
    const bool al = aligned16(x) && aligned16(y);
    const unsigned nrows = (unsigned)rows;
    switch (al ? pick_block_p(c) : 0) {
    case 1: softmax_block_kernel<1><<<nrows, kBlockThreads, 0, s>>>(x, y, c); return;
    case 2: softmax_block_kernel<2><<<nrows, kBlockThreads, 0, s>>>(x, y, c); return;
    case 4: softmax_block_kernel<4><<<nrows, kBlockThreads, 0, s>>>(x, y, c); return;
    case 8: softmax_block_kernel<8><<<nrows, kBlockThreads, 0, s>>>(x, y, c); return;
    case 16: softmax_block_kernel<16><<<nrows, kBlockThreads, 0, s>>>(x, y, c); return;
    default: break;
    }
    const int vpt = al ? pick_vpt(c) : 0;
    switch (vpt) {
    case 1: softmax_wave_kernel<1><<<grid, 256, 0, s>>>(x, y, r, c); break;
    case 2: softmax_wave_kernel<2><<<grid, 256, 0, s>>>(x, y, r, c); break;
    case 4: softmax_wave_kernel<4><<<grid, 256, 0, s>>>(x, y, r, c); break;
    case 8: softmax_wave_kernel<8><<<grid, 256, 0, s>>>(x, y, r, c); break;
    case 16: softmax_wave_kernel<16><<<grid, 256, 0, s>>>(x, y, r, c); break;
    case 32: softmax_wave_kernel<32><<<grid, 256, 0, s>>>(x, y, r, c); break;
    default: softmax_loop_kernel<<<grid, 256, 0, s>>>(x, y, r, c); break;
    }
}

void layer_norm_rows(const float *x, const float *gamma, const float *beta, float *y,
                     size_t rows, size_t cols, float eps, hipStream_t s) {
    if (!rows || !cols) return;
    const unsigned grid = (unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock);
    const int r = (int)rows, c = (int)cols;
    const bool al = aligned16(x) && aligned16(y) && aligned16(gamma) && aligned16(beta);
    const int vpt = al ? pick_vpt(c) : 0;
    const size_t lds = 2 * (size_t)c * sizeof(float);
    switch (vpt) {
    case 1: layer_norm_wave_kernel<1><<<grid, 256, lds, s>>>(x, gamma, beta, y, r, c, eps); break;
    case 2: layer_norm_wave_kernel<2><<<grid, 256, lds, s>>>(x, gamma, beta, y, r, c, eps); break;
    case 4: layer_norm_wave_kernel<4><<<grid, 256, lds, s>>>(x, gamma, beta, y, r, c, eps); break;
    case 8: layer_norm_wave_kernel<8><<<grid, 256, lds, s>>>(x, gamma, beta, y, r, c, eps); break;
    case 16: layer_norm_wave_kernel<16><<<grid, 256, lds, s>>>(x, gamma, beta, y, r, c, eps); break;
    case 32: layer_norm_wave_kernel<32><<<grid, 256, lds, s>>>(x, gamma, beta, y, r, c, eps); break;
    default: layer_norm_loop_kernel<<<grid, 256, 0, s>>>(x, gamma, beta, y, r, c, eps); break;
    }
}

void softmax_backward_rows(const float *y, const float *dy, float *dx, size_t rows, size_t cols,
                           hipStream_t s) {
    if (!rows || !cols) return;
    const unsigned grid = (unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock);
    const int r = (int)rows, c = (int)cols;
    const bool al = aligned16(y) && aligned16(dy) && aligned16(dx);
    const unsigned nrows = (unsigned)rows;
    switch (al ? pick_block_p(c) : 0) {
    case 1: softmax_bw_block_kernel<1><<<nrows, kBlockThreads, 0, s>>>(y, dy, dx, c); return;
    case 2: softmax_bw_block_kernel<2><<<nrows, kBlockThreads, 0, s>>>(y, dy, dx, c); return;
    case 4: softmax_bw_block_kernel<4><<<nrows, kBlockThreads, 0, s>>>(y, dy, dx, c); return;
    case 8: softmax_bw_block_kernel<8><<<nrows, kBlockThreads, 0, s>>>(y, dy, dx, c); return;
    case 16: softmax_bw_block_kernel<16><<<nrows, kBlockThreads, 0, s>>>(y, dy, dx, c); return;
    default: break;
    }
    const int vpt = al ? pick_vpt(c) : 0;
    switch (vpt) {
    case 1: softmax_bw_wave_kernel<1><<<grid, 256, 0, s>>>(y, dy, dx, r, c); break;
    case 2: softmax_bw_wave_kernel<2><<<grid, 256, 0, s>>>(y, dy, dx, r, c); break;
    case 4: softmax_bw_wave_kernel<4><<<grid, 256, 0, s>>>(y, dy, dx, r, c); break;
    case 8: softmax_bw_wave_kernel<8><<<grid, 256, 0, s>>>(y, dy, dx, r, c); break;
    case 16: softmax_bw_wave_kernel<16><<<grid, 256, 0, s>>>(y, dy, dx, r, c); break;
    default: softmax_bw_loop_kernel<<<grid, 256, 0, s>>>(y, dy, dx, r, c); break;
    }
}

template <int MODE>
static void cross_entropy_launch(const float *logits, const float *targets, size_t used,
                                 size_t rows, size_t cols, const float *grad_loss, float *out,
                                 int *err_flag, hipStream_t s) {
    const unsigned grid = (unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock);
    const int r = (int)rows, c = (int)cols;
    const long u = (long)used;
    const bool al = aligned16(logits) && (MODE == 0 || aligned16(out));
    const unsigned nrows = (unsigned)rows;
    if (MODE == 0 && al && (pick_block_p(c) == 1 || pick_block_p(c) == 2)) {
        const unsigned pairs = (unsigned)((rows + 1) / 2);
        if (pick_block_p(c) == 1)
            cross_entropy_rows2_kernel<1><<<pairs, kBlockThreads, 0, s>>>(logits, targets, u, r, c, out, err_flag);
        else
            cross_entropy_rows2_kernel<2><<<pairs, kBlockThreads, 0, s>>>(logits, targets, u, r, c, out, err_flag);
        return;
    }
    switch (al ? pick_block_p(c) : 0) {
    case 1: cross_entropy_block_kernel<1, MODE><<<nrows, kBlockThreads, 0, s>>>(logits, targets, u, r, c, grad_loss, out, err_flag); return;
    case 2: cross_entropy_block_kernel<2, MODE><<<nrows, kBlockThreads, 0, s>>>(logits, targets, u, r, c, grad_loss, out, err_flag); return;
    case 4: cross_entropy_block_kernel<4, MODE><<<nrows, kBlockThreads, 0, s>>>(logits, targets, u, r, c, grad_loss, out, err_flag); return;
    case 8: cross_entropy_block_kernel<8, MODE><<<nrows, kBlockThreads, 0, s>>>(logits, targets, u, r, c, grad_loss, out, err_flag); return;
    case 16: cross_entropy_block_kernel<16, MODE><<<nrows, kBlockThreads, 0, s>>>(logits, targets, u, r, c, grad_loss, out, err_flag); return;
    default: break;
    }
    const int vpt = al ? pick_vpt(c) : 0;
    switch (vpt) {
    case 1: cross_entropy_wave_kernel<1, MODE><<<grid, 256, 0, s>>>(logits, targets, u, r, c, grad_loss, out, err_flag); break;
    case 2: cross_entropy_wave_kernel<2, MODE><<<grid, 256, 0, s>>>(logits, targets, u, r, c, grad_loss, out, err_flag); break;
    case 4: cross_entropy_wave_kernel<4, MODE><<<grid, 256, 0, s>>>(logits, targets, u, r, c, grad_loss, out, err_flag); break;
    case 8: cross_entropy_wave_kernel<8, MODE><<<grid, 256, 0, s>>>(logits, targets, u, r, c, grad_loss, out, err_flag); break;
    case 16: cross_entropy_wave_kernel<16, MODE><<<grid, 256, 0, s>>>(logits, targets, u, r, c, grad_loss, out, err_flag); break;
    default: cross_entropy_loop_kernel<MODE><<<grid, 256, 0, s>>>(logits, targets, u, r, c, grad_loss, out, err_flag); break;
    }
}

void cross_entropy_rows(const float *logits, const float *targets, size_t used, size_t rows,
                        size_t cols, float *row_values, int *err_flag, hipStream_t s) {
    if (!rows || !cols) return;
    cross_entropy_launch<0>(logits, targets, used, rows, cols, nullptr, row_values, err_flag, s);
}

void cross_entropy_backward_rows(const float *logits, const float *targets, size_t used,
                                 size_t rows, size_t cols, const float *grad_loss, float *grad,
                                 int *err_flag, hipStream_t s) {
    if (!rows || !cols) return;
    cross_entropy_launch<1>(logits, targets, used, rows, cols, grad_loss, grad, err_flag, s);
}

}  // namespace k
}  // namespace clove
