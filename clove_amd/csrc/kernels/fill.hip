// fill.hip -- seeded synthetic data on the device.
//
// Element i of a stream with seed s is derived from a splitmix64 hash of a
// Weyl sequence: z(j) = mix64(s + (j + 1) * 0x9E3779B97F4A7C15), where mix64
// is the splitmix64 finaliser (Steele, Lea and Flood, "Fast splittable
// pseudorandom number generators", 2014).  The top 24 bits of z give a
// uniform in [0, 1).  Normals use the Box-Muller pair of (2j, 2j+1):
// r = sqrt(-2 ln u1), theta = 2 pi u2 with u1 in (0, 1]; element 2j takes
// r cos theta and element 2j+1 takes r sin theta.  The integer part is exact
// on any platform; the transcendental part rounds like the device library.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "launch.hpp"

namespace clove {
namespace k {

namespace {

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t stream_at(uint64_t seed, uint64_t j) {
    return mix64(seed + (j + 1) * 0x9E3779B97F4A7C15ull);
}

__global__ void __launch_bounds__(256) fill_uniform_kernel(float *p, uint64_t n, uint64_t seed,
                                                           float lo, float hi) {
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * 256) {
        const float u = (float)(stream_at(seed, i) >> 40) * 0x1p-24f;
        p[i] = lo + (hi - lo) * u;
    }
}

__global__ void __launch_bounds__(256) fill_normal_kernel(float *p, uint64_t n, uint64_t seed,
                                                          float mean, float stddev) {
    const uint64_t pairs = (n + 1) / 2;
    for (uint64_t j = (uint64_t)blockIdx.x * 256 + threadIdx.x; j < pairs;
         j += (uint64_t)gridDim.x * 256) {
        const float u1 = (float)((stream_at(seed, 2 * j) >> 40) + 1) * 0x1p-24f;
        const float u2 = (float)(stream_at(seed, 2 * j + 1) >> 40) * 0x1p-24f;
        const float r = sqrtf(-2.0f * logf(u1));
        const float th = 6.2831853071795865f * u2;
        p[2 * j] = mean + stddev * (r * cosf(th));
        if (2 * j + 1 < n) p[2 * j + 1] = mean + stddev * (r * sinf(th));
    }
}

unsigned grid_for(uint64_t work) {
    uint64_t b = (work + 255) / 256;
    if (b > 65536) b = 65536;
    return b ? (unsigned)b : 1u;
}

}  // namespace

void fill_normal(float *p, size_t n, uint64_t seed, float mean, float stddev, hipStream_t s) {
    if (!n) return;
    fill_normal_kernel<<<grid_for((n + 1) / 2), 256, 0, s>>>(p, n, seed, mean, stddev);
}

void fill_uniform(float *p, size_t n, uint64_t seed, float lo, float hi, hipStream_t s) {
    if (!n) return;
    fill_uniform_kernel<<<grid_for(n), 256, 0, s>>>(p, n, seed, lo, hi);
}

}  // namespace k
}  // namespace clove
