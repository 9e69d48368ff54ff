// probe_hbm_floor -- what a 64 MiB HBM-bound step can reach on MI355X when
// its input is cold, i.e. not in the 256 MB last-level cache (not part of
// the library; `make -C clove_amd/csrc probe` builds it).
//
// Part 1: g [4096, 4096] f32 (64 MiB) in eight copies cycled from launch to
// launch (512 MiB: the last-level cache cannot keep them).  Each workgroup
// sums W contiguous bytes of every row of its row range and stores its
// partial column sums (no combine), for W from a 128-byte piece to the whole
// 16 KiB row, at 128 to 512 workgroups (128 also with 512 threads each:
// twice the loads in flight per CU); it prints the time per launch and
// the read rate against the 8 TB/s peak.  With three copies instead (192
// MiB, all of them in the cache) the same launches read far faster.
// Part 2: the cost of a dependent second launch: a writer of n floats
// followed by a one-workgroup fixed-order sum of them (1024 threads, or one
// wave with 16-byte loads), against the writer alone.
// Every access is in bounds (indices checked against the allocations below)
// and every loop has a fixed trip count.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>

#define CK(x)                                                                        \
    do {                                                                             \
        hipError_t e_ = (x);                                                         \
        if (e_ != hipSuccess) {                                                      \
            std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
            std::exit(1);                                                            \
        }                                                                            \
    } while (0)

typedef float f4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int kRows = 4096, kCols = 4096, kQuads = kCols / 4;
constexpr size_t kPartBytes = (size_t)64 << 20;

// Q 16-byte quads of a row per workgroup, T threads: thread (q, rg) sums quad
// q over rows rg, rg + T/Q, ... of [r0, r0 + rows_per), eight loads at a time.
template <int Q, int T>
__global__ void __launch_bounds__(T) strip_sums(const float *g, float *part, int rows_per) {
    constexpr int RG = T / Q, KB = 8;
    const int strips = kQuads / Q;
    const int sidx = blockIdx.x % strips, seg = blockIdx.x / strips;
    const int ql = threadIdx.x % Q, rg = threadIdx.x / Q;
    const int q = sidx * Q + ql;
    const int r0 = seg * rows_per, r1 = r0 + rows_per;
    const f4 *g4 = reinterpret_cast<const f4 *>(g);
    f4 s = {0.f, 0.f, 0.f, 0.f};
    for (int r = r0 + rg; r < r1; r += RG * KB) {
        f4 v[KB];
#pragma unroll
        for (int u = 0; u < KB; ++u) {
            const int rr = r + u * RG;
            v[u] = rr < r1 ? g4[(size_t)rr * kQuads + q] : (f4){0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int u = 0; u < KB; ++u) s += v[u];
    }
    // index < segs * RG * kQuads quads: segs * RG <= 256 in main(), so at
    // most 256 x 1024 quads x 16 B = 4 MiB, inside part
    reinterpret_cast<f4 *>(part)[((size_t)seg * RG + rg) * kQuads + q] = s;
}

template <int Q, int T>
void launch_strips(const float *g, float *part, int segs) {
    strip_sums<Q, T><<<(kQuads / Q) * segs, T>>>(g, part, kRows / segs);
}

__global__ void writer(float *x, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) x[i] = 1.0f + (float)(i % 7) * 0.25f;
}

__device__ __forceinline__ float wave_sum(float v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// one workgroup of 1024 threads, eight loads per thread, wave sums in LDS
__global__ void __launch_bounds__(1024) sum_block(const float *x, int n, float *out) {
    __shared__ float ws[16];
    float s = 0.f;
    for (int base = threadIdx.x; base < n; base += 8 * 1024) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int i = base + u * 1024;
            v[u] = i < n ? x[i] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) s += v[u];
    }
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = ws[0];
        for (int w = 1; w < 16; ++w) t += ws[w];
        out[0] = t / (float)n;
    }
}

// one wave, 16-byte loads (n a multiple of 4), 32 in flight per lane
__global__ void __launch_bounds__(64) sum_wave(const float *x, int n, float *out) {
    const f4 *x4 = reinterpret_cast<const f4 *>(x);
    const int nv = n / 4;
    float s = 0.f;
    for (int base = threadIdx.x; base < nv; base += 64 * 32) {
        f4 v[32];
#pragma unroll
        for (int u = 0; u < 32; ++u) {
            const int i = base + 64 * u;
            v[u] = i < nv ? x4[i] : (f4){0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int u = 0; u < 32; ++u) s += (v[u].x + v[u].y) + (v[u].z + v[u].w);
    }
    s = wave_sum(s);
    if (threadIdx.x == 0) out[0] = s / (float)n;
}

struct StripCase {
    const char *name;
    void (*fn)(const float *, float *, int);
    int segs;
};

double time_strips(const StripCase &c, float *const *g, int copies, float *part) {
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    for (int i = 0; i < 24; ++i) c.fn(g[i % copies], part, c.segs);
    CK(hipGetLastError());
    constexpr int kN = 200;
    CK(hipEventRecord(e0));
    for (int i = 0; i < kN; ++i) c.fn(g[i % copies], part, c.segs);
    CK(hipEventRecord(e1));
    CK(hipEventSynchronize(e1));
    float ms = 0.f;
    CK(hipEventElapsedTime(&ms, e0, e1));
    CK(hipEventDestroy(e0));
    CK(hipEventDestroy(e1));
    return ms * 1e3 / kN;
}

}  // namespace

int main() {
    constexpr int kCopies = 8;
    const size_t bytes = (size_t)kRows * kCols * 4;
    float *g[kCopies], *part, *x, *out;
    for (int i = 0; i < kCopies; ++i) {
        CK(hipMalloc(&g[i], bytes));
        CK(hipMemset(g[i], 0, bytes));
    }
    CK(hipMalloc(&part, kPartBytes));
    // part 1: Q quads per row x T threads x segments; segs * (T / Q) <= 256
    // rows of partials of 4096 floats, at most 4 MiB
    const StripCase cases[] = {
        {"128 B pieces, 128 workgroups", launch_strips<8, 256>, 1},
        {"128 B pieces, 128 x 512 thr.", launch_strips<8, 512>, 1},
        {"128 B pieces, 256 workgroups", launch_strips<8, 256>, 2},
        {"512 B pieces, 256 workgroups", launch_strips<32, 256>, 8},
        {"2 KiB pieces, 256 workgroups", launch_strips<128, 256>, 32},
        {"2 KiB pieces, 512 workgroups", launch_strips<128, 256>, 64},
        {"16 KiB rows,  256 workgroups", launch_strips<1024, 1024>, 256},
    };
    std::printf("part 1: a 64 MiB read, g [4096, 4096] f32, column sums per workgroup\n");
    for (const StripCase &c : cases)
        for (int copies : {kCopies, 3}) {
            const double us = time_strips(c, g, copies, part);
            std::printf("  %-30s %d copies (%4d MiB): %6.2f us  %5.1f%% of 8 TB/s\n", c.name,
                        copies, copies * 64, us, 100.0 * bytes / (us * 1e-6) / 8e12);
            std::fflush(stdout);
        }

    // part 2: the second, dependent launch
    constexpr int kN = 8192;
    CK(hipMalloc(&x, kN * 4));
    CK(hipMalloc(&out, 64));
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    const char *names[] = {"writer alone", "writer + 1024-thread sum", "writer + one-wave sum"};
    double base_us = 0.0;
    std::printf("part 2: a writer of %d floats, then a fixed-order sum of them\n", kN);
    for (int which = 0; which < 3; ++which) {
        auto step = [&] {
            writer<<<(kN + 255) / 256, 256>>>(x, kN);
            if (which == 1) sum_block<<<1, 1024>>>(x, kN, out);
            if (which == 2) sum_wave<<<1, 64>>>(x, kN, out);
        };
        for (int i = 0; i < 20; ++i) step();
        constexpr int kSteps = 500;
        CK(hipEventRecord(e0));
        for (int i = 0; i < kSteps; ++i) step();
        CK(hipEventRecord(e1));
        CK(hipEventSynchronize(e1));
        float ms = 0.f;
        CK(hipEventElapsedTime(&ms, e0, e1));
        const double us = ms * 1e3 / kSteps;
        if (which == 0) base_us = us;
        double mean = 0.0;
        for (int i = 0; i < kN; ++i) mean += 1.0 + (i % 7) * 0.25;
        mean /= kN;
        float h = 0.f;
        if (which) CK(hipMemcpy(&h, out, 4, hipMemcpyDeviceToHost));
        std::printf("  %-26s %6.2f us per step (+%.2f us)%s\n", names[which], us, us - base_us,
                    which && std::fabs(h - mean) > 1e-5 ? "  WRONG SUM" : "");
        std::fflush(stdout);
    }
    return 0;
}
