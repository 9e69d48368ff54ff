// ew_chain_kernel.h -- skeleton of a fused elementwise chain kernel.
//
// The runtime-generated source defines, before including this file:
//   CL_NIN, CL_NOUT          number of inputs and of stored values
//   cl_load_all<T>(a, i, x)  loads every input at vector/element i into x[]
//   cl_body<T>(x, prm, y)    the chain itself, T = float or cl_f4
//   CL_KERNEL_NAME           the kernel's symbol (it names the chain's ops,
//                            so profiles show which chain ran)
// Each thread streams CL_UNROLL 16-byte vectors per input per iteration
// (all loads issued before any arithmetic), walking the index space with a
// grid stride; a scalar loop finishes the elements past the last full vector.
// CL_BLOCK and CL_UNROLL come from the generator (512 threads, two vectors:
// a block covers 16 KiB of each input, read by eight waves at once).
#pragma once

#ifndef CL_UNROLL
#define CL_UNROLL 4
#endif
#ifndef CL_BLOCK
#define CL_BLOCK 256
#endif

extern "C" __global__ void __launch_bounds__(CL_BLOCK) CL_KERNEL_NAME(cl_chain_args a) {
    const unsigned long long nvec = a.nvec;
    const unsigned long long tile = (unsigned long long)CL_BLOCK * CL_UNROLL;
    const unsigned long long stride = (unsigned long long)gridDim.x * tile;
    for (unsigned long long base = (unsigned long long)blockIdx.x * tile + threadIdx.x;
         base < nvec; base += stride) {
        if (base + (CL_UNROLL - 1) * (unsigned long long)CL_BLOCK < nvec) {
            cl_f4 x[CL_UNROLL][CL_NIN];
#pragma unroll
            for (int u = 0; u < CL_UNROLL; ++u) cl_load_all(a, base + u * CL_BLOCK, x[u]);
#pragma unroll
            for (int u = 0; u < CL_UNROLL; ++u) {
                cl_f4 y[CL_NOUT];
                cl_body(x[u], a.param, y);
#pragma unroll
                for (int o = 0; o < CL_NOUT; ++o) cl_store4(a.out[o], base + u * CL_BLOCK, y[o]);
            }
        } else {
            for (int u = 0; u < CL_UNROLL; ++u) {
                const unsigned long long v = base + u * CL_BLOCK;
                if (v < nvec) {
                    cl_f4 x[CL_NIN], y[CL_NOUT];
                    cl_load_all(a, v, x);
                    cl_body(x, a.param, y);
#pragma unroll
                    for (int o = 0; o < CL_NOUT; ++o) cl_store4(a.out[o], v, y[o]);
                }
            }
        }
    }
    for (unsigned long long i = 4ull * nvec + (unsigned long long)blockIdx.x * CL_BLOCK + threadIdx.x;
         i < a.numel; i += (unsigned long long)gridDim.x * CL_BLOCK) {
        float x[CL_NIN], y[CL_NOUT];
        cl_load_all(a, i, x);
        cl_body(x, a.param, y);
#pragma unroll
        for (int o = 0; o < CL_NOUT; ++o) a.out[o][i] = y[o];
    }
}
