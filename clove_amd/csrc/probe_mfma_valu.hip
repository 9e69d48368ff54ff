// probe_mfma_valu -- measures whether VALU work overlaps FP32 MFMAs on one
// SIMD (not part of the library; `make -C clove_amd/csrc probe` builds it).
//
// Part 1: one wave issues 1024 independent v_mfma_f32_32x32x2_f32 (four
// accumulators, or one for a dependent chain) with NV plain VALU ops or NT
// v_exp_f32 placed after each MFMA of its own.
// Part 2: eight waves in one workgroup (two per SIMD): waves 0-3 issue the
// same MFMA stream alone while waves 4-7 run NV VALU ops per MFMA-time step.
// Each prints the MFMA waves' shader-clock cycles per MFMA (s_memtime).
// Every access is in bounds (one float per thread, one 64-bit count) and
// every loop has a fixed trip count.
#include <hip/hip_runtime.h>

#include <cstdio>

typedef float f16v __attribute__((ext_vector_type(16)));

template <int NV, int NT, int NA>
__global__ void __launch_bounds__(64) own_wave(float *out, long long *cyc, float x0) {
    f16v acc[4];
    for (int j = 0; j < 4; ++j)
        for (int e = 0; e < 16; ++e) acc[j][e] = 0.f;
    const float a = x0 + threadIdx.x, b = x0 * 2.f;
    float v[8];
    for (int i = 0; i < 8; ++i) v[i] = x0 + i;
    const long long t0 = clock64();
    for (int it = 0; it < 64; ++it) {
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            acc[k % NA] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[k % NA], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < NV; ++i) v[i & 7] = v[i & 7] * 1.0001f + 0.5f;
#pragma unroll
            for (int i = 0; i < NT; ++i) v[i & 7] = __builtin_amdgcn_exp2f(v[i & 7]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    const long long t1 = clock64();
    float s = 0.f;
    for (int j = 0; j < 4; ++j)
        for (int e = 0; e < 16; ++e) s += acc[j][e];
    for (int i = 0; i < 8; ++i) s += v[i];
    out[threadIdx.x] = s;
    if (threadIdx.x == 0) cyc[0] = t1 - t0;
}

template <int NV>
__global__ void __launch_bounds__(512) other_wave(float *out, long long *cyc, float x0) {
    const int wave = threadIdx.x >> 6;
    float s = 0.f;
    if (wave < 4) {
        f16v acc[4];
        for (int j = 0; j < 4; ++j)
            for (int e = 0; e < 16; ++e) acc[j][e] = 0.f;
        const float a = x0 + threadIdx.x, b = x0 * 2.f;
        const long long t0 = clock64();
        for (int it = 0; it < 64; ++it) {
#pragma unroll
            for (int k = 0; k < 16; ++k)
                acc[k & 3] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[k & 3], 0, 0, 0);
        }
        const long long t1 = clock64();
        for (int j = 0; j < 4; ++j)
            for (int e = 0; e < 16; ++e) s += acc[j][e];
        if (threadIdx.x == 0) cyc[0] = t1 - t0;
    } else {
        float v[8];
        for (int i = 0; i < 8; ++i) v[i] = x0 + i;
        for (int it = 0; it < 64 * 16; ++it) {
#pragma unroll
            for (int i = 0; i < NV; ++i) v[i & 7] = v[i & 7] * 1.0001f + 0.5f;
        }
        for (int i = 0; i < 8; ++i) s += v[i];
    }
    out[threadIdx.x] = s;
}

static float *g_out;
static long long *g_cyc;

static double cycles_per_mfma() {
    long long h = 0;
    (void)hipMemcpy(&h, g_cyc, sizeof h, hipMemcpyDeviceToHost);
    return h / 1024.0;
}

template <int NV, int NT, int NA = 4>
static void run_own() {
    for (int rep = 0; rep < 2; ++rep) own_wave<NV, NT, NA><<<1, 64>>>(g_out, g_cyc, 0.001f);
    printf("own wave:   accumulators %d, %2d VALU + %d v_exp after each MFMA: %6.1f cycles/MFMA\n",
           NA, NV, NT, cycles_per_mfma());
}

template <int NV>
static void run_other() {
    for (int rep = 0; rep < 2; ++rep) other_wave<NV><<<1, 512>>>(g_out, g_cyc, 0.001f);
    printf("other wave: %2d VALU per MFMA-time step on the same SIMD:          %6.1f cycles/MFMA\n",
           NV, cycles_per_mfma());
}

int main() {
    if (hipMalloc(&g_out, 512 * sizeof(float)) != hipSuccess ||
        hipMalloc(&g_cyc, sizeof(long long)) != hipSuccess) {
        fprintf(stderr, "hipMalloc failed\n");
        return 1;
    }
    run_own<0, 0>();
    run_own<0, 0, 1>();
    run_own<2, 0>();
    run_own<4, 0>();
    run_own<8, 0>();
    run_own<16, 0>();
    run_own<0, 2>();
    run_own<0, 4>();
    run_other<0>();
    run_other<4>();
    run_other<8>();
    run_other<16>();
    (void)hipFree(g_out);
    (void)hipFree(g_cyc);
    return 0;
}
