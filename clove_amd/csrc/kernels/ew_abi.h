// ew_abi.h -- argument layout shared by the host launcher (jit.cpp) and the
// fused-chain kernels compiled at run time.  Plain C++: no device code.
#pragma once

#define CL_MAX_IN 16
#define CL_MAX_OUT 16
#define CL_MAX_OPS 48

// Operand k of a chain is read as input_k[idx % numel_k] (lazy.rs:1600-1608,
// backend.rs:1489).  The host classifies each operand once per launch and
// the classification is part of the compiled chain's signature.
enum {
    CL_BCAST_FULL = 0,    // numel_k == numel(out): element idx
    CL_BCAST_SCALAR = 1,  // numel_k == 1: element 0
    CL_BCAST_MODVEC = 2,  // numel_k % 4 == 0: four contiguous elements at idx % numel_k
    CL_BCAST_MODELEM = 3  // anything else: one modulo per element
};

struct cl_operand {
    const float *p;
    unsigned long long n;  // numel_k
    unsigned int magic;    // 32-bit division magic for n (valid when n < 2^32)
    unsigned int shift;
};

struct cl_chain_args {
    cl_operand in[CL_MAX_IN];
    float *out[CL_MAX_OUT];
    float param[CL_MAX_OPS];
    unsigned long long numel;  // elements in the output index space
    unsigned long long nvec;   // vectors of 4 handled by the vector path
};
