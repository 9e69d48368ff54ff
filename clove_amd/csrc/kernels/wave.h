// wave.h -- wave64 reductions and small device helpers shared by the
// ahead-of-time kernels.
#pragma once

#include <hip/hip_runtime.h>

typedef float cl_f4 __attribute__((ext_vector_type(4)));

// Butterfly reductions across the 64 lanes of a wavefront; every lane ends
// with the result, and the combination order is fixed (deterministic).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Reduction over the 32 lanes of each half of the wavefront.
__device__ __forceinline__ float half_sum(float v) {
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float hmax4(cl_f4 v) { return fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w)); }
__device__ __forceinline__ float hsum4(cl_f4 v) { return (v.x + v.y) + (v.z + v.w); }
