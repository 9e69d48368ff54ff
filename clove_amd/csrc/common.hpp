// common.hpp -- shared host-side types of the HIP backend: status handling,
// the tensor record behind a CTensor handle, and the device context.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/clove_hip.h"

namespace clove {

// Errors travel as exceptions inside the library and become status codes at
// the C ABI (capi.cpp); nothing escapes extern "C" functions.
struct Error {
    int code;
    std::string msg;
};

[[noreturn]] void fail(int code, const std::string &msg);
void set_last_error(const std::string &msg);

#define CLOVE_HIP_CHECK(expr)                                                          \
    do {                                                                               \
        hipError_t e_ = (expr);                                                        \
        if (e_ != hipSuccess)                                                          \
            ::clove::fail(CLOVE_HIP_ERR_HIP, std::string(#expr) + ": " + hipGetErrorString(e_)); \
    } while (0)

#define CLOVE_REQUIRE(cond, code, msg)      \
    do {                                    \
        if (!(cond)) ::clove::fail(code, msg); \
    } while (0)

// One device allocation plus its logical shape: the data half of Clove's
// TensorGraph (tensor.rs:77-84).  Autograd fields are out of scope.
struct Tensor {
    void *data = nullptr;
    std::vector<size_t> shape;
    int dtype = CLOVE_HIP_F32;
    size_t numel = 0;
    size_t bytes = 0;     // capacity of the allocation
    bool owned = true;    // false for clove_hip_tensor_wrap views

    Tensor() = default;
    Tensor(const Tensor &) = delete;
    Tensor &operator=(const Tensor &) = delete;
    ~Tensor();

    float *f32() const { return static_cast<float *>(data); }
    int32_t *i32() const { return static_cast<int32_t *>(data); }
    size_t dim(int i) const { return shape[i < 0 ? shape.size() + i : i]; }
};

// Shared ownership mirrors TensorNode = Arc<RwLock<TensorGraph>> (tensor.rs:67).
using TensorNode = std::shared_ptr<Tensor>;

size_t numel_of(const std::vector<size_t> &shape);
std::string shape_str(const std::vector<size_t> &shape);

// Allocates a device tensor through the caching allocator.
TensorNode new_tensor(const std::vector<size_t> &shape, int dtype);

// ---- device context ------------------------------------------------------

struct Context {
    int device = -1;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;  // own_stream unless a caller stream is set
    int num_cus = 0;
    int num_xcds = 8;
    size_t l2_bytes = 0;
    std::string arch;
};

Context &ctx();            // fails with CLOVE_HIP_ERR_NOT_INIT before init
bool ctx_ready();
std::recursive_mutex &api_mutex();

// Caching allocator (stream-ordered on the single stream: a block freed after
// kernels were enqueued is only reused by work enqueued later on that stream).
void *dev_alloc(size_t bytes, size_t *capacity);
void dev_free(void *p, size_t capacity);
void dev_empty_cache();
size_t dev_reserved();

}  // namespace clove
