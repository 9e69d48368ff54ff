// runtime.cpp -- device context, caching allocator, tensor records, events.
//
// Replaces the wgpu glue of the reference: EngineDevice::init
// (device.rs:79-150) becomes clove_hip_init on one HIP device with one
// stream; wgpu buffers become caching-allocator blocks; map_async readback
// (backend.rs:1056-1090) becomes hipMemcpyAsync + stream sync.
#include <cstring>
#include <map>
#include <unordered_map>

#include "common.hpp"
#include "kernels/launch.hpp"
#include "runtime.hpp"

namespace clove {

namespace {
thread_local std::string g_last_error;
Context g_ctx;
bool g_ready = false;

// Free blocks by capacity.  Capacities are size classes, so a request only
// reuses a block of its own class.  Created once and never destroyed: tensors
// held by other translation units' statics (the RoPE table cache) are
// released by their destructors at process exit, in an order the language
// leaves open, and must still find a live map to return their blocks to.
std::multimap<size_t, void *> &free_blocks() {
    static auto *m = new std::multimap<size_t, void *>();
    return *m;
}
size_t g_reserved = 0;

std::vector<hipEvent_t> g_events;

int32_t *g_err_flag = nullptr;  // device word set by kernels that saw bad indices

// Device address of the paged decode's static scratch array, per device
// ordinal (each GPU holds its own copy of the array at its own address).
constexpr int kMaxDevices = 64;
float *g_paged_scratch[kMaxDevices] = {};
}  // namespace

void set_last_error(const std::string &msg) { g_last_error = msg; }
const std::string &last_error() { return g_last_error; }

void fail(int code, const std::string &msg) { throw Error{code, msg}; }

std::recursive_mutex &api_mutex() {
    static auto *m = new std::recursive_mutex();  // never destroyed (see free_blocks)
    return *m;
}

Context &ctx() {
    if (!g_ready) fail(CLOVE_HIP_ERR_NOT_INIT, "clove_hip_init has not been called");
    return g_ctx;
}
bool ctx_ready() { return g_ready; }

size_t numel_of(const std::vector<size_t> &shape) {
    size_t n = 1;
    for (size_t d : shape) n *= d;
    return n;
}

std::string shape_str(const std::vector<size_t> &shape) {
    std::string s = "[";
    for (size_t i = 0; i < shape.size(); ++i) {
        if (i) s += ", ";
        s += std::to_string(shape[i]);
    }
    return s + "]";
}

// ---- allocator -----------------------------------------------------------

static size_t size_class(size_t bytes) {
    if (bytes == 0) bytes = 1;
    if (bytes <= (1u << 20)) {
        size_t c = 512;
        while (c < bytes) c <<= 1;
        return c;
    }
    const size_t gran = 2u << 20;
    return (bytes + gran - 1) / gran * gran;
}

void *dev_alloc(size_t bytes, size_t *capacity) {
    ctx();  // fails before clove_hip_init
    const size_t cap = size_class(bytes);
    auto it = free_blocks().find(cap);
    if (it != free_blocks().end()) {
        void *p = it->second;
        free_blocks().erase(it);
        *capacity = cap;
        return p;
    }
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, cap);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        dev_empty_cache();
        e = hipMalloc(&p, cap);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            fail(CLOVE_HIP_ERR_OOM, "hipMalloc of " + std::to_string(cap) + " bytes failed: " +
                                        hipGetErrorString(e));
        }
    }
    g_reserved += cap;
    *capacity = cap;
    return p;
}

void dev_free(void *p, size_t capacity) {
    if (!p) return;
    free_blocks().emplace(capacity, p);
}

void dev_empty_cache() {
    if (free_blocks().empty()) return;
    // Blocks may still be referenced by enqueued kernels.
    (void)hipStreamSynchronize(g_ctx.stream);
    for (auto &kv : free_blocks()) {
        (void)hipFree(kv.second);
        g_reserved -= kv.first;
    }
    free_blocks().clear();
}

size_t dev_reserved() { return g_reserved; }

// ---- tensors -------------------------------------------------------------

Tensor::~Tensor() {
    if (owned && data && g_ready) {
        std::lock_guard<std::recursive_mutex> lk(api_mutex());
        dev_free(data, bytes);
    }
}

TensorNode new_tensor(const std::vector<size_t> &shape, int dtype) {
    CLOVE_REQUIRE(dtype == CLOVE_HIP_F32 || dtype == CLOVE_HIP_I32, CLOVE_HIP_ERR_INVALID,
                  "unknown dtype " + std::to_string(dtype));
    auto t = std::make_shared<Tensor>();
    t->shape = shape;
    t->dtype = dtype;
    t->numel = numel_of(shape);
    t->data = dev_alloc(t->numel * 4, &t->bytes);
    return t;
}

// ---- context -------------------------------------------------------------

void init(int device) {
    if (g_ready) {
        CLOVE_REQUIRE(device == g_ctx.device, CLOVE_HIP_ERR_INVALID,
                      "already initialised on device " + std::to_string(g_ctx.device));
        return;
    }
    int count = 0;
    CLOVE_HIP_CHECK(hipGetDeviceCount(&count));
    CLOVE_REQUIRE(device >= 0 && device < count, CLOVE_HIP_ERR_INVALID,
                  "device ordinal " + std::to_string(device) + " out of range (" +
                      std::to_string(count) + " devices)");
    CLOVE_HIP_CHECK(hipSetDevice(device));
    CLOVE_REQUIRE(device < kMaxDevices, CLOVE_HIP_ERR_INVALID, "device ordinal too large");
    if (!g_paged_scratch[device]) {
        // with `device` current: the address of this GPU's copy
        float *p = nullptr;
        CLOVE_HIP_CHECK(k::paged_scratch_address(&p));
        CLOVE_REQUIRE(p != nullptr, CLOVE_HIP_ERR_HIP, "no address for the paged scratch array");
        g_paged_scratch[device] = p;
    }
    hipDeviceProp_t prop;
    CLOVE_HIP_CHECK(hipGetDeviceProperties(&prop, device));
    std::string arch = prop.gcnArchName;
    CLOVE_REQUIRE(arch.rfind("gfx950", 0) == 0, CLOVE_HIP_ERR_INVALID,
                  "this backend is built for gfx950 (MI355X); device reports " + arch);
    g_ctx.device = device;
    g_ctx.arch = arch;
    g_ctx.num_cus = prop.multiProcessorCount;
    g_ctx.l2_bytes = (size_t)prop.l2CacheSize;
    CLOVE_HIP_CHECK(hipStreamCreateWithFlags(&g_ctx.own_stream, hipStreamNonBlocking));
    g_ctx.stream = g_ctx.own_stream;
    g_ready = true;
    size_t cap = 0;
    g_err_flag = static_cast<int32_t *>(dev_alloc(4, &cap));
    CLOVE_HIP_CHECK(hipMemsetAsync(g_err_flag, 0, 4, g_ctx.stream));
    CLOVE_HIP_CHECK(hipStreamSynchronize(g_ctx.stream));
}

void shutdown() {
    if (!g_ready) return;
    (void)hipStreamSynchronize(g_ctx.stream);
    jit_shutdown();
    rope_cache_clear();
    for (hipEvent_t e : g_events) (void)hipEventDestroy(e);
    g_events.clear();
    dev_empty_cache();
    if (g_err_flag) {
        (void)hipFree(g_err_flag);
        g_reserved -= 512;
        g_err_flag = nullptr;
    }
    (void)hipStreamDestroy(g_ctx.own_stream);
    g_ctx = Context{};
    g_ready = false;
}

int32_t *device_error_flag() {
    ctx();
    return g_err_flag;
}

float *paged_scratch() { return g_paged_scratch[ctx().device]; }


void synchronize() {
    Context &c = ctx();
    CLOVE_HIP_CHECK(hipStreamSynchronize(c.stream));
    int32_t flag = 0;
    CLOVE_HIP_CHECK(hipMemcpy(&flag, g_err_flag, 4, hipMemcpyDeviceToHost));
    if (flag) {
        CLOVE_HIP_CHECK(hipMemset(g_err_flag, 0, 4));
        std::string msg = "an earlier call met an index out of range:";
        if (flag & k::kErrPagedRange)
            msg += " a block-table entry outside the KV pool or a context length past the "
                   "table (those tokens were skipped);";
        if (flag & k::kErrClassRange)
            msg += " a cross-entropy target >= the number of classes (that row counted 0);";
        if (flag & k::kErrIndexValue)
            msg += " an f32 block_tables/context_lens value that is not an integer in "
                   "[0, 2^24) (read as -1: its tokens were skipped);";
        msg.pop_back();
        fail(CLOVE_HIP_ERR_RANGE, msg);
    }
}

void set_stream(void *s) {
    Context &c = ctx();
    CLOVE_HIP_CHECK(hipStreamSynchronize(c.stream));
    c.stream = s ? static_cast<hipStream_t>(s) : c.own_stream;
}

// ---- host <-> device -----------------------------------------------------

void upload(Tensor &t, const void *src, size_t offset, size_t count) {
    CLOVE_REQUIRE(offset + count <= t.numel, CLOVE_HIP_ERR_RANGE,
                  "write of [" + std::to_string(offset) + ", " + std::to_string(offset + count) +
                      ") past numel " + std::to_string(t.numel));
    if (!count) return;
    Context &c = ctx();
    CLOVE_HIP_CHECK(hipMemcpyAsync(static_cast<char *>(t.data) + offset * 4, src, count * 4,
                                   hipMemcpyHostToDevice, c.stream));
    CLOVE_HIP_CHECK(hipStreamSynchronize(c.stream));
}

void download(const Tensor &t, void *dst, size_t offset, size_t count) {
    CLOVE_REQUIRE(offset + count <= t.numel, CLOVE_HIP_ERR_RANGE,
                  "read of [" + std::to_string(offset) + ", " + std::to_string(offset + count) +
                      ") past numel " + std::to_string(t.numel));
    Context &c = ctx();
    if (count)
        CLOVE_HIP_CHECK(hipMemcpyAsync(dst, static_cast<const char *>(t.data) + offset * 4,
                                       count * 4, hipMemcpyDeviceToHost, c.stream));
    synchronize();
}

// ---- events --------------------------------------------------------------

int event_record() {
    Context &c = ctx();
    hipEvent_t e;
    CLOVE_HIP_CHECK(hipEventCreate(&e));
    CLOVE_HIP_CHECK(hipEventRecord(e, c.stream));
    g_events.push_back(e);
    return (int)g_events.size() - 1;
}

float event_elapsed(int a, int b) {
    CLOVE_REQUIRE(a >= 0 && b >= 0 && a < (int)g_events.size() && b < (int)g_events.size(),
                  CLOVE_HIP_ERR_INVALID, "unknown event id");
    CLOVE_HIP_CHECK(hipEventSynchronize(g_events[b]));
    float ms = 0.f;
    CLOVE_HIP_CHECK(hipEventElapsedTime(&ms, g_events[a], g_events[b]));
    return ms;
}

void event_reset() {
    for (hipEvent_t e : g_events) (void)hipEventDestroy(e);
    g_events.clear();
}

}  // namespace clove
