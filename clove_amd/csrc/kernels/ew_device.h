// ew_device.h -- elementwise semantics of Clove's hot-path ops on gfx950.
//
// This header is compiled into every fused chain that the library builds at
// run time with hipRTC (jit.cpp embeds its text), so it uses only clang
// builtins and the device math that hipRTC provides.
//
// Rounding: chains are compiled with -ffp-contract=off so every expression
// rounds exactly as Clove's Rayon kernels do (Rust never contracts a*b+c into
// an FMA); transcendental calls use the ROCm device library (expf, tanhf,
// sinf, cosf), which differs from glibc by at most a few ulp.
#pragma once

#include "ew_abi.h"

typedef float cl_f4 __attribute__((ext_vector_type(4)));

// sqrt(2/pi) evaluated in f32 the way backend.rs:1924 does,
// (2.0f32 / PI).sqrt() == 0x3F4C4229.  (The lazy WGSL at lazy.rs:1761 writes
// the literal 0.7978845608, one ulp higher; parity is with the CPU path.)
#define CL_GELU_K 0x1.988452p-1f

// ---- scalar op semantics -------------------------------------------------

__device__ __forceinline__ float cl_add(float a, float b) { return a + b; }   // backend.rs:1490
__device__ __forceinline__ float cl_sub(float a, float b) { return a - b; }   // backend.rs:1755
__device__ __forceinline__ float cl_mul(float a, float b) { return a * b; }   // backend.rs:1608-1613
__device__ __forceinline__ float cl_relu(float x) { return x > 0.0f ? x : 0.0f; }  // backend.rs:1823
__device__ __forceinline__ float cl_gelu(float x) {                              // backend.rs:1924-1925
    const float x3 = (x * x) * x;  // powi(3)
    const float inner = CL_GELU_K * (x + 0.044715f * x3);
    return 0.5f * x * (1.0f + tanhf(inner));
}
__device__ __forceinline__ float cl_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }  // backend.rs:2958
__device__ __forceinline__ float cl_tanh(float x) { return tanhf(x); }  // backend.rs:3015
__device__ __forceinline__ float cl_sin(float x) { return sinf(x); }    // backend.rs:1994
__device__ __forceinline__ float cl_cos(float x) { return cosf(x); }    // backend.rs:2052
__device__ __forceinline__ float cl_scale(float x, float s) { return x * s; }  // backend.rs:1694
// ReluGrad(x, g): select(0, g, x > 0) (lazy.rs:1757-1763)
__device__ __forceinline__ float cl_relu_grad(float x, float g) { return x > 0.0f ? g : 0.0f; }
// GeluGrad(x, g): derivative of the tanh-form GELU times g (fused WGSL
// lazy.rs:1764-1779; CPU backward backend.rs:1965-1981, whose rounding this
// follows: 3.0 * 0.044715 is folded in f32 first and meets x*x as one
// operand, 0.5 * x * sech2 * c * (...) is evaluated left to right).
__device__ __forceinline__ float cl_gelu_grad(float x, float g) {
    const float x3 = (x * x) * x;
    const float t = tanhf(CL_GELU_K * (x + 0.044715f * x3));
    const float sech2 = 1.0f - t * t;
    const float d = 0.5f * (1.0f + t) +
                    0.5f * x * sech2 * CL_GELU_K * (1.0f + (3.0f * 0.044715f) * (x * x));
    return g * d;
}

// ---- the same ops on 4-wide vectors (componentwise) -----------------------

#define CL_VEC1(name)                                                             \
    __device__ __forceinline__ cl_f4 name(cl_f4 v) {                              \
        return (cl_f4){name(v.x), name(v.y), name(v.z), name(v.w)};               \
    }
#define CL_VEC2(name)                                                             \
    __device__ __forceinline__ cl_f4 name(cl_f4 a, cl_f4 b) {                     \
        return (cl_f4){name(a.x, b.x), name(a.y, b.y), name(a.z, b.z), name(a.w, b.w)}; \
    }
CL_VEC2(cl_add)
CL_VEC2(cl_sub)
CL_VEC2(cl_mul)
CL_VEC1(cl_relu)
CL_VEC1(cl_gelu)
CL_VEC1(cl_sigmoid)
CL_VEC1(cl_tanh)
CL_VEC1(cl_sin)
CL_VEC1(cl_cos)
CL_VEC2(cl_relu_grad)
CL_VEC2(cl_gelu_grad)
__device__ __forceinline__ cl_f4 cl_scale(cl_f4 v, float s) {
    return (cl_f4){v.x * s, v.y * s, v.z * s, v.w * s};
}

// ---- broadcast operand loads ----------------------------------------------

// x % n for x, n < 2^32 with a precomputed magic multiplier (Granlund and
// Montgomery, "Division by invariant integers using multiplication", 1994,
// Fig. 4.1): q = (t + ((x - t) >> 1)) >> (l - 1), t = mulhi(m, x).
__device__ __forceinline__ unsigned int cl_mod32(unsigned int x, const cl_operand &o) {
    const unsigned int t = __umulhi(x, o.magic);
    const unsigned int q = (t + ((x - t) >> 1)) >> o.shift;
    return x - q * (unsigned int)o.n;
}

template <bool WIDE>
__device__ __forceinline__ unsigned long long cl_mod(unsigned long long x, const cl_operand &o) {
    if (WIDE) return x % o.n;
    return (unsigned long long)cl_mod32((unsigned int)x, o);
}

// Vector v covers elements 4v .. 4v+3 of the output index space.
template <int MODE, bool WIDE>
__device__ __forceinline__ cl_f4 cl_load4(const cl_operand &o, unsigned long long v) {
    if (MODE == CL_BCAST_FULL) {
        return __builtin_nontemporal_load(reinterpret_cast<const cl_f4 *>(o.p) + v);
    } else if (MODE == CL_BCAST_SCALAR) {
        const float s = o.p[0];
        return (cl_f4){s, s, s, s};
    } else if (MODE == CL_BCAST_MODVEC) {
        return *reinterpret_cast<const cl_f4 *>(o.p + cl_mod<WIDE>(4ull * v, o));
    } else {
        const unsigned long long i = 4ull * v;
        return (cl_f4){o.p[cl_mod<WIDE>(i, o)], o.p[cl_mod<WIDE>(i + 1, o)],
                       o.p[cl_mod<WIDE>(i + 2, o)], o.p[cl_mod<WIDE>(i + 3, o)]};
    }
}

template <int MODE, bool WIDE>
__device__ __forceinline__ float cl_load1(const cl_operand &o, unsigned long long i) {
    if (MODE == CL_BCAST_FULL) return o.p[i];
    if (MODE == CL_BCAST_SCALAR) return o.p[0];
    return o.p[cl_mod<WIDE>(i, o)];
}

__device__ __forceinline__ void cl_store4(float *p, unsigned long long v, cl_f4 x) {
    __builtin_nontemporal_store(x, reinterpret_cast<cl_f4 *>(p) + v);
}
