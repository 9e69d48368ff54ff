// optim.hip -- the fused AdamW update (optim.rs:305-345 WGSL, 375-395 CPU).
//
// One pass per element: decoupled weight decay, loss-scale unscaling and
// clipping, both moments, bias correction and the step, reading w, g, m, v
// and writing w, m, v (28 bytes per element, HBM-bound).  Up to kMaxTensors
// parameter tensors go in one launch (grid y = tensor), so a model's many
// small parameters do not each pay a launch; their pointers and sizes travel
// in the kernel arguments, so no device-side table is allocated.
//
// Rounding follows the CPU branch exactly: built with -ffp-contract=off,
// IEEE division and square root (HIP's defaults for f32), Rust's operand
// order, and 1 - beta^t computed on the host with the same powf.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "launch.hpp"
#include "wave.h"

namespace clove {
namespace k {

namespace {

struct AdamWArgs {
    float *w[kAdamWMaxTensors];
    const float *g[kAdamWMaxTensors];
    float *m[kAdamWMaxTensors];
    float *v[kAdamWMaxTensors];
    uint64_t n[kAdamWMaxTensors];
    AdamWHyper h;
};

// Rust's f32::clamp: NaN passes through.
__device__ __forceinline__ float clamp_rs(float x, float lo, float hi) {
    if (x < lo) x = lo;
    if (x > hi) x = hi;
    return x;
}

__device__ __forceinline__ void adamw_elem(float &w, float g, float &m, float &v,
                                           const AdamWHyper &h) {
    w -= h.lr * h.weight_decay * w;
    const float gc = clamp_rs(g / h.loss_scale, -h.clip, h.clip);
    m = h.beta1 * m + (1.0f - h.beta1) * gc;
    v = h.beta2 * v + (1.0f - h.beta2) * gc * gc;
    const float m_hat = m / h.bias1;
    const float v_hat = v / h.bias2;
    w -= h.lr * m_hat / (sqrtf(v_hat) + h.eps);
}

// 512-thread workgroups, every load and store non-temporal: with the steps
// cycling through parameter copies that the 256 MB last-level cache cannot
// hold, 4096 x 4096 took 76.9-78.0 us (75-76% of HBM peak) against 87.7-89.2
// us with ordinary loads and stores for w, m and v and a 16-per-CU grid cap
// (80.7 us non-temporal at that cap; caps of 24-64 and 256-thread groups
// within 2 us).  Ordinary accesses led (83.9% against 75.5%) only while one
// 256 MiB copy was updated every step and that cache kept part of it.
constexpr int kAdamWThreads = 512;
__global__ void __launch_bounds__(kAdamWThreads) adamw_kernel(AdamWArgs a) {
    const int t = blockIdx.y;
    const uint64_t n = a.n[t];
    float *__restrict__ w = a.w[t];
    const float *__restrict__ g = a.g[t];
    float *__restrict__ m = a.m[t];
    float *__restrict__ v = a.v[t];
    const uint64_t stride = (uint64_t)gridDim.x * kAdamWThreads;
    // 16-byte vectors when all four arrays are aligned; the rest element-wise
    const bool vec = ((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(g) |
                       reinterpret_cast<uintptr_t>(m) | reinterpret_cast<uintptr_t>(v)) & 15) == 0;
    const uint64_t nvec = vec ? n / 4 : 0;
    for (uint64_t i = (uint64_t)blockIdx.x * kAdamWThreads + threadIdx.x; i < nvec; i += stride) {
        cl_f4 wv = __builtin_nontemporal_load(reinterpret_cast<cl_f4 *>(w) + i);
        const cl_f4 gv = __builtin_nontemporal_load(reinterpret_cast<const cl_f4 *>(g) + i);
        cl_f4 mv = __builtin_nontemporal_load(reinterpret_cast<cl_f4 *>(m) + i);
        cl_f4 vv = __builtin_nontemporal_load(reinterpret_cast<cl_f4 *>(v) + i);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            float wc = wv[c], mc = mv[c], vc = vv[c];
            adamw_elem(wc, gv[c], mc, vc, a.h);
            wv[c] = wc;
            mv[c] = mc;
            vv[c] = vc;
        }
        __builtin_nontemporal_store(wv, reinterpret_cast<cl_f4 *>(w) + i);
        __builtin_nontemporal_store(mv, reinterpret_cast<cl_f4 *>(m) + i);
        __builtin_nontemporal_store(vv, reinterpret_cast<cl_f4 *>(v) + i);
    }
    for (uint64_t i = 4 * nvec + (uint64_t)blockIdx.x * kAdamWThreads + threadIdx.x; i < n;
         i += stride) {
        float wc = w[i], mc = m[i], vc = v[i];
        adamw_elem(wc, g[i], mc, vc, a.h);
        w[i] = wc;
        m[i] = mc;
        v[i] = vc;
    }
}

}  // namespace

void adamw_step(float *const *w, const float *const *g, float *const *m, float *const *v,
                const uint64_t *n, int count, const AdamWHyper &h, int num_cus, hipStream_t s) {
    for (int base = 0; base < count; base += kAdamWMaxTensors) {
        const int c = count - base < kAdamWMaxTensors ? count - base : kAdamWMaxTensors;
        AdamWArgs a{};
        uint64_t most = 0;
        for (int j = 0; j < c; ++j) {
            a.w[j] = w[base + j];
            a.g[j] = g[base + j];
            a.m[j] = m[base + j];
            a.v[j] = v[base + j];
            a.n[j] = n[base + j];
            if (n[base + j] > most) most = n[base + j];
        }
        a.h = h;
        if (!most) continue;
        // enough workgroups for the largest tensor (4 elements per thread per
        // pass), capped at 32 per CU and tensor: the loop strides the rest
        uint64_t blocks = (most / 4 + kAdamWThreads - 1) / kAdamWThreads;
        const uint64_t cap = (uint64_t)num_cus * 32 / (uint64_t)c;
        if (blocks > cap) blocks = cap > 0 ? cap : 1;
        if (blocks < 1) blocks = 1;
        adamw_kernel<<<dim3((unsigned)blocks, (unsigned)c), kAdamWThreads, 0, s>>>(a);
    }
}

}  // namespace k
}  // namespace clove
