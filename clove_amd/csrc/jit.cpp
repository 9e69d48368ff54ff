// jit.cpp -- runtime code generation for fused elementwise chains.
//
// The MI355X counterpart of Clove's `flush_fused` WGSL generator
// (lazy.rs:1694-1838): a chain of elementwise IR nodes becomes one kernel.
// The generated source is a short HIP body (one line per op) dropped into a
// fixed kernel skeleton (kernels/ew_chain_kernel.h) that streams 16-byte
// vectors; it is compiled for gfx950 with hipRTC, loaded with
// hipModuleLoadData and launched with hipModuleLaunchKernel.  Kernels are
// cached by signature: the op structure plus each input's broadcast class.
// Op parameters (ScalarMul factors, dropout scales) are kernel arguments, so
// they never cause a recompile.
//
// Differences from the reference generator, on purpose:
//   - every op with `store` set is written, not only the last one
//     (lazy.rs:1823 drops intermediates that escape the group);
//   - an opcode the generator does not know is an error, not silently
//     skipped (lazy.rs:1820 `_ => {}`);
//   - indices are 64-bit and vectorised; the reference dispatches one thread
//     per element with 32-bit indices and a `%` per operand per element.
#include <hip/hiprtc.h>
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <sstream>
#include <unordered_map>

#include "common.hpp"
#include "kernels/ew_abi.h"
#include "runtime.hpp"

namespace clove {

namespace {

const char kAbiSrc[] =
#include "ew_abi.inc"
    ;
const char kDeviceSrc[] =
#include "ew_device.inc"
    ;
const char kKernelSrc[] =
#include "ew_chain_kernel.inc"
    ;

struct Compiled {
    hipModule_t module = nullptr;
    hipFunction_t fn = nullptr;
};

std::unordered_map<std::string, Compiled> g_cache;

// Launch-geometry knobs for tuning sweeps: CLOVE_CHAIN_UNROLL (vectors per
// thread per input per iteration, default 2), CLOVE_CHAIN_BLOCK (threads per
// block, 64-1024 in steps of 64, default 512) and CLOVE_CHAIN_BLOCKS_PER_CU
// (grid cap, default 32).  They change scheduling only, never the result.
// The defaults were the fastest of a sweep with inputs and outputs cycled so
// the last-level cache held neither (config 2's chain, one box): 512 x 2 gave
// 76.5% of HBM peak and 77.7-79.0% on the broadcast chain, against 74.1% /
// 75.9% for 512 x 1, 75.1% for 512 x 3, 72.5% for 512 x 4, 76.2% for
// 1024 x 2 and 75.8% for 256 x 4; caps of 16 and 64 blocks per CU measured
// as 32.  (Rewriting one output block every step, 512 x 1 read 79.9%: the
// last-level cache then keeps part of the output.)
int env_int(const char *name, int dflt, int lo, int hi) {
    const char *v = std::getenv(name);
    if (!v || !*v) return dflt;
    const int x = std::atoi(v);
    return x < lo ? lo : (x > hi ? hi : x);
}
int chain_unroll() { return env_int("CLOVE_CHAIN_UNROLL", 2, 1, 16); }
int chain_block() { return (env_int("CLOVE_CHAIN_BLOCK", 512, 64, 1024) / 64) * 64; }
int chain_blocks_per_cu() { return env_int("CLOVE_CHAIN_BLOCKS_PER_CU", 32, 1, 1024); }

const char *op_fn(int opcode) {
    switch (opcode) {
    case CLOVE_OP_ADD: return "cl_add";
    case CLOVE_OP_SUB: return "cl_sub";
    case CLOVE_OP_MUL: return "cl_mul";
    case CLOVE_OP_RELU: return "cl_relu";
    case CLOVE_OP_GELU: return "cl_gelu";
    case CLOVE_OP_SIN: return "cl_sin";
    case CLOVE_OP_COS: return "cl_cos";
    case CLOVE_OP_SIGMOID: return "cl_sigmoid";
    case CLOVE_OP_TANH: return "cl_tanh";
    case CLOVE_OP_RELU_GRAD: return "cl_relu_grad";
    case CLOVE_OP_GELU_GRAD: return "cl_gelu_grad";
    case CLOVE_OP_SCALAR_MUL:
    case CLOVE_OP_DROPOUT: return "cl_scale";
    default: return nullptr;
    }
}

// Granlund-Montgomery magic for 32-bit unsigned division by d >= 1:
// l = ceil(log2 d), m = floor(2^32 (2^l - d) / d) + 1, shift = l - 1.
void division_magic(uint64_t d, unsigned int *magic, unsigned int *shift) {
    if (d <= 1 || d > 0xFFFFFFFFull) {
        *magic = 0;
        *shift = 0;
        return;
    }
    unsigned int l = 0;
    while ((1ull << l) < d) ++l;
    const uint64_t m = ((1ull << 32) * ((1ull << l) - d)) / d + 1;
    *magic = (unsigned int)m;
    *shift = l - 1;
}

// Kernel symbol naming the chain, e.g. clove_chain_mul_add_gelu_mul_b0000
// (the suffix lists each input's broadcast class).
std::string kernel_name(const std::vector<ChainOp> &ops, const std::vector<int> &modes) {
    static const char *names[] = {"input", "matmul", "add", "sub", "mul", "scale", "flatten",
                                  "relu", "gelu", "sin", "cos", "softmax", "layernorm",
                                  "dropout", "relugrad", "gelugrad", "cast", "sigmoid", "tanh"};
    std::string n = "clove_chain";
    for (size_t i = 0; i < ops.size() && i < 12; ++i) {
        const int op = ops[i].opcode;
        n += "_";
        n += (op >= 0 && op < (int)(sizeof(names) / sizeof(names[0]))) ? names[op] : "op";
    }
    if (ops.size() > 12) n += "_more";
    n += "_b";
    for (int m : modes) n += char('0' + m);
    return n;
}

std::string operand_expr(int src) {
    return src < 0 ? "x[" + std::to_string(-src - 1) + "]" : "n" + std::to_string(src);
}

std::string generate(const std::vector<ChainOp> &ops, const std::vector<int> &modes, bool wide,
                     int nout, const std::string &name, int unroll, int block) {
    std::ostringstream s;
    const int nin = (int)modes.size();
    s << "#define CL_NIN " << nin << "\n#define CL_NOUT " << nout << "\n";
    s << "#define CL_KERNEL_NAME " << name << "\n#define CL_UNROLL " << unroll << "\n";
    s << "#define CL_BLOCK " << block << "\n";
    s << "#include \"ew_device.h\"\n";
    s << "__device__ __forceinline__ void cl_load_all(const cl_chain_args &a, unsigned long long v, cl_f4 *x) {\n";
    for (int k = 0; k < nin; ++k)
        s << "    x[" << k << "] = cl_load4<" << modes[k] << ", " << (wide ? "true" : "false")
          << ">(a.in[" << k << "], v);\n";
    s << "}\n";
    s << "__device__ __forceinline__ void cl_load_all(const cl_chain_args &a, unsigned long long i, float *x) {\n";
    for (int k = 0; k < nin; ++k)
        s << "    x[" << k << "] = cl_load1<" << modes[k] << ", " << (wide ? "true" : "false")
          << ">(a.in[" << k << "], i);\n";
    s << "}\n";
    s << "template <typename T>\n__device__ __forceinline__ void cl_body(const T *x, const float *prm, T *y) {\n";
    int o = 0;
    for (size_t i = 0; i < ops.size(); ++i) {
        const ChainOp &op = ops[i];
        const std::string dst = "n" + std::to_string(i);
        const std::string a0 = operand_expr(op.src0);
        switch (op.opcode) {
        case CLOVE_OP_FLATTEN:
        case CLOVE_OP_CAST:
            s << "    const T " << dst << " = " << a0 << ";\n";
            break;
        case CLOVE_OP_SCALAR_MUL:
        case CLOVE_OP_DROPOUT:
            s << "    const T " << dst << " = cl_scale(" << a0 << ", prm[" << i << "]);\n";
            break;
        default:
            if (ew_arity(op.opcode) == 2)
                s << "    const T " << dst << " = " << op_fn(op.opcode) << "(" << a0 << ", "
                  << operand_expr(op.src1) << ");\n";
            else
                s << "    const T " << dst << " = " << op_fn(op.opcode) << "(" << a0 << ");\n";
        }
        if (op.store || i + 1 == ops.size()) s << "    y[" << o++ << "] = " << dst << ";\n";
    }
    s << "    (void)prm;\n}\n#include \"ew_chain_kernel.h\"\n";
    return s.str();
}

std::string signature(const std::vector<ChainOp> &ops, const std::vector<int> &modes, bool wide) {
    std::ostringstream s;
    for (size_t i = 0; i < ops.size(); ++i)
        s << ops[i].opcode << '(' << ops[i].src0 << ',' << ops[i].src1 << ')'
          << ((ops[i].store || i + 1 == ops.size()) ? "s" : "") << ';';
    s << "|m";
    for (int m : modes) s << m;
    s << (wide ? "|w" : "|n");
    s << "|u" << chain_unroll() << "|t" << chain_block();
    return s.str();
}

const char *const kRtcOpts[] = {"--offload-arch=gfx950", "-O3", "-ffp-contract=off", "-std=c++17",
                                // no packed-f32 instructions in any device code of this library
                                "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
constexpr int kNumRtcOpts = (int)(sizeof(kRtcOpts) / sizeof(kRtcOpts[0]));

int g_compiles = 0, g_disk_loads = 0;

// ---- code objects on disk -------------------------------------------------
// A chain compiled once is kept as a code object under CLOVE_JIT_CACHE (a
// directory; "0" or "off" turns the cache off), by default
// $XDG_CACHE_HOME/clove_hip or $HOME/.cache/clove_hip, so a new process
// loads it instead of running hipRTC again (tens to hundreds of ms per
// chain).  The file holds the whole key -- generated source, the embedded
// headers, the compile options and the hipRTC, HIP runtime and driver
// versions -- and is used only if that key matches exactly, so a changed
// library or toolchain never loads a stale object.  A 64-bit checksum of the
// code bytes catches a damaged file.  Only a regular file owned by this user
// and writable by no one else is read, and it is opened without following
// symbolic links, so a file another user planted in a shared directory is
// never loaded.  New directories are created 0700; files are written to a
// fresh temporary name (O_EXCL, random suffix, 0600) and renamed, so a
// reader never sees a partial one.  Any failure to read, load or write just
// means compiling.
const char kCacheMagic[8] = {'C', 'L', 'V', 'J', 'I', 'T', '0', '2'};

std::string cache_dir() {
    const char *v = std::getenv("CLOVE_JIT_CACHE");
    if (v) {
        if (!*v || !std::strcmp(v, "0") || !std::strcmp(v, "off")) return "";
        return v;
    }
    if (const char *x = std::getenv("XDG_CACHE_HOME"); x && *x) return std::string(x) + "/clove_hip";
    if (const char *h = std::getenv("HOME"); h && *h) return std::string(h) + "/.cache/clove_hip";
    return "";
}

std::string cache_key(const std::string &src) {
    int maj = 0, min = 0, rt = 0, drv = 0;
    hiprtcVersion(&maj, &min);
    (void)hipRuntimeGetVersion(&rt);
    (void)hipDriverGetVersion(&drv);
    std::string k = src;
    for (const char *h : {kAbiSrc, kDeviceSrc, kKernelSrc}) k += std::string("\x01") + h;
    for (int i = 0; i < kNumRtcOpts; ++i) k += std::string("\x02") + kRtcOpts[i];
    k += "\x03hiprtc " + std::to_string(maj) + "." + std::to_string(min) + " runtime " +
         std::to_string(rt) + " driver " + std::to_string(drv) + " arch " + ctx().arch;
    return k;
}

uint64_t fnv1a(const char *p, size_t n) {
    uint64_t h = 1469598103934665603ull;
    for (size_t i = 0; i < n; ++i) h = (h ^ (unsigned char)p[i]) * 1099511628211ull;
    return h;
}

std::string cache_path(const std::string &dir, const std::string &key) {
    char name[32];
    std::snprintf(name, sizeof(name), "%016llx.co",
                  (unsigned long long)fnv1a(key.data(), key.size()));
    return dir + "/" + name;
}

bool read_all(int fd, void *dst, size_t n) {
    char *p = static_cast<char *>(dst);
    while (n) {
        const ssize_t r = read(fd, p, n);
        if (r <= 0) return false;
        p += r;
        n -= (size_t)r;
    }
    return true;
}

bool write_all(int fd, const void *src, size_t n) {
    const char *p = static_cast<const char *>(src);
    while (n) {
        const ssize_t r = write(fd, p, n);
        if (r <= 0) return false;
        p += r;
        n -= (size_t)r;
    }
    return true;
}

bool cache_read(const std::string &path, const std::string &key, std::vector<char> *code) {
    const int fd = open(path.c_str(), O_RDONLY | O_NOFOLLOW | O_CLOEXEC);
    if (fd < 0) return false;
    struct stat st;
    bool ok = fstat(fd, &st) == 0 && S_ISREG(st.st_mode) && st.st_uid == geteuid() &&
              (st.st_mode & (S_IWGRP | S_IWOTH)) == 0;
    char magic[8];
    uint64_t klen = 0, clen = 0, sum = 0;
    ok = ok && read_all(fd, magic, 8) && !std::memcmp(magic, kCacheMagic, 8) &&
         read_all(fd, &klen, 8) && klen == key.size();
    if (ok) {
        std::string k(klen, '\0');
        ok = read_all(fd, &k[0], klen) && k == key && read_all(fd, &clen, 8) && clen > 0 &&
             clen < (256u << 20) && read_all(fd, &sum, 8);
        if (ok) {
            code->resize(clen);
            ok = read_all(fd, code->data(), clen) && fnv1a(code->data(), clen) == sum;
        }
    }
    close(fd);
    return ok;
}

void cache_write(const std::string &dir, const std::string &path, const std::string &key,
                 const std::vector<char> &code) {
    for (size_t i = 1; i <= dir.size(); ++i)  // mkdir -p
        if (i == dir.size() || dir[i] == '/') (void)mkdir(dir.substr(0, i).c_str(), 0700);
    std::random_device rd;
    char suffix[40];
    std::snprintf(suffix, sizeof(suffix), ".tmp%ld.%08x%08x", (long)getpid(), rd(), rd());
    const std::string tmp = path + suffix;
    const int fd = open(tmp.c_str(), O_WRONLY | O_CREAT | O_EXCL | O_NOFOLLOW | O_CLOEXEC, 0600);
    if (fd < 0) return;
    const uint64_t klen = key.size(), clen = code.size(), sum = fnv1a(code.data(), clen);
    const bool ok = write_all(fd, kCacheMagic, 8) && write_all(fd, &klen, 8) &&
                    write_all(fd, key.data(), klen) && write_all(fd, &clen, 8) &&
                    write_all(fd, &sum, 8) && write_all(fd, code.data(), clen);
    if (close(fd) != 0 || !ok || std::rename(tmp.c_str(), path.c_str()) != 0)
        (void)std::remove(tmp.c_str());
}

Compiled load_code(const std::vector<char> &code, const std::string &name) {
    Compiled c;
    CLOVE_HIP_CHECK(hipModuleLoadData(&c.module, code.data()));
    CLOVE_HIP_CHECK(hipModuleGetFunction(&c.fn, c.module, name.c_str()));
    return c;
}

// A cached object whose key matched but that the runtime will not load
// (damaged on disk) is not fatal: the caller compiles and rewrites it.
bool try_load_code(const std::vector<char> &code, const std::string &name, Compiled *c) {
    if (hipModuleLoadData(&c->module, code.data()) != hipSuccess) return false;
    if (hipModuleGetFunction(&c->fn, c->module, name.c_str()) != hipSuccess) {
        (void)hipModuleUnload(c->module);
        return false;
    }
    return true;
}

Compiled compile(const std::string &src, const std::string &name) {
    const std::string dir = cache_dir();
    std::string key, path;
    if (!dir.empty()) {
        key = cache_key(src);
        path = cache_path(dir, key);
        std::vector<char> code;
        Compiled c;
        if (cache_read(path, key, &code) && try_load_code(code, name, &c)) {
            ++g_disk_loads;
            return c;
        }
    }
    hiprtcProgram prog;
    const char *headers[] = {kAbiSrc, kDeviceSrc, kKernelSrc};
    const char *names[] = {"ew_abi.h", "ew_device.h", "ew_chain_kernel.h"};
    if (hiprtcCreateProgram(&prog, src.c_str(), "clove_chain.hip", 3, headers, names) !=
        HIPRTC_SUCCESS)
        fail(CLOVE_HIP_ERR_JIT, "hiprtcCreateProgram failed");
    hiprtcResult r = hiprtcCompileProgram(prog, kNumRtcOpts, kRtcOpts);
    if (r != HIPRTC_SUCCESS) {
        size_t n = 0;
        hiprtcGetProgramLogSize(prog, &n);
        std::string log(n, '\0');
        if (n) hiprtcGetProgramLog(prog, &log[0]);
        hiprtcDestroyProgram(&prog);
        fail(CLOVE_HIP_ERR_JIT, std::string("hipRTC compile failed: ") + log + "\n--- source ---\n" + src);
    }
    size_t code_size = 0;
    hiprtcGetCodeSize(prog, &code_size);
    std::vector<char> code(code_size);
    hiprtcGetCode(prog, code.data());
    hiprtcDestroyProgram(&prog);
    ++g_compiles;
    Compiled c = load_code(code, name);
    if (!dir.empty()) cache_write(dir, path, key, code);
    return c;
}

}  // namespace

int ew_arity(int opcode) {
    switch (opcode) {
    case CLOVE_OP_ADD:
    case CLOVE_OP_SUB:
    case CLOVE_OP_MUL:
    case CLOVE_OP_RELU_GRAD:
    case CLOVE_OP_GELU_GRAD:
        return 2;
    case CLOVE_OP_SCALAR_MUL:
    case CLOVE_OP_FLATTEN:
    case CLOVE_OP_RELU:
    case CLOVE_OP_GELU:
    case CLOVE_OP_SIN:
    case CLOVE_OP_COS:
    case CLOVE_OP_DROPOUT:
    case CLOVE_OP_CAST:
    case CLOVE_OP_SIGMOID:
    case CLOVE_OP_TANH:
        return 1;
    default:
        return 0;
    }
}

int validate_chain(const std::vector<ChainOp> &ops, size_t n_inputs) {
    CLOVE_REQUIRE(!ops.empty(), CLOVE_HIP_ERR_INVALID, "empty chain");
    CLOVE_REQUIRE((int)ops.size() <= CL_MAX_OPS, CLOVE_HIP_ERR_INVALID,
                  "chain longer than " + std::to_string(CL_MAX_OPS) + " ops");
    CLOVE_REQUIRE(n_inputs <= (size_t)CL_MAX_IN && n_inputs > 0, CLOVE_HIP_ERR_INVALID,
                  "a chain takes 1.." + std::to_string(CL_MAX_IN) + " inputs");
    int nstore = 0;
    for (size_t i = 0; i < ops.size(); ++i) {
        const ChainOp &op = ops[i];
        const int ar = ew_arity(op.opcode);
        CLOVE_REQUIRE(ar > 0, CLOVE_HIP_ERR_INVALID,
                      "opcode " + std::to_string(op.opcode) + " is not elementwise");
        const int srcs[2] = {op.src0, op.src1};
        for (int j = 0; j < ar; ++j) {
            // 64-bit, so that -(src + 1) of INT_MIN does not overflow
            const int64_t s = srcs[j];
            const bool earlier_op = s >= 0 && s < (int64_t)i;
            const bool input = s < 0 && -s - 1 < (int64_t)n_inputs;
            CLOVE_REQUIRE(earlier_op || input, CLOVE_HIP_ERR_INVALID,
                          "op " + std::to_string(i) + " operand " + std::to_string(s) +
                              " is neither an earlier op nor an input");
        }
        if (op.store || i + 1 == ops.size()) ++nstore;
    }
    CLOVE_REQUIRE(nstore <= CL_MAX_OUT, CLOVE_HIP_ERR_INVALID,
                  "chain stores " + std::to_string(nstore) + " values; at most " +
                      std::to_string(CL_MAX_OUT) + " are allowed");
    return nstore;
}

void run_chain(const std::vector<ChainOp> &ops, const std::vector<const Tensor *> &inputs,
               const std::vector<Tensor *> &outs, size_t numel) {
    Context &c = ctx();
    const int nstore = validate_chain(ops, inputs.size());
    CLOVE_REQUIRE(nstore == (int)outs.size(), CLOVE_HIP_ERR_INVALID,
                  "chain stores " + std::to_string(nstore) + " values but " +
                      std::to_string(outs.size()) + " outputs were given");
    if (numel == 0) return;

    const bool wide = numel > 0xFFFFFFFFull;
    cl_chain_args args;
    std::memset(&args, 0, sizeof(args));
    std::vector<int> modes(inputs.size());
    bool aligned = true;
    for (size_t k = 0; k < inputs.size(); ++k) {
        const Tensor *t = inputs[k];
        CLOVE_REQUIRE(t && t->dtype == CLOVE_HIP_F32, CLOVE_HIP_ERR_INVALID,
                      "chain input " + std::to_string(k) + " must be an f32 tensor");
        CLOVE_REQUIRE(t->numel > 0, CLOVE_HIP_ERR_SHAPE,
                      "chain input " + std::to_string(k) + " is empty");
        const uint64_t n = t->numel;
        int m;
        if (n >= numel) m = CL_BCAST_FULL;
        else if (n == 1) m = CL_BCAST_SCALAR;
        else if (n % 4 == 0) m = CL_BCAST_MODVEC;
        else m = CL_BCAST_MODELEM;
        modes[k] = m;
        args.in[k].p = t->f32();
        args.in[k].n = n;
        division_magic(n, &args.in[k].magic, &args.in[k].shift);
        if ((reinterpret_cast<uintptr_t>(t->data) & 15) != 0 &&
            (m == CL_BCAST_FULL || m == CL_BCAST_MODVEC))
            aligned = false;
    }
    for (size_t o = 0; o < outs.size(); ++o) {
        CLOVE_REQUIRE(outs[o]->dtype == CLOVE_HIP_F32 && outs[o]->numel >= numel,
                      CLOVE_HIP_ERR_SHAPE, "chain output too small");
        args.out[o] = outs[o]->f32();
        if ((reinterpret_cast<uintptr_t>(outs[o]->data) & 15) != 0) aligned = false;
    }
    for (size_t i = 0; i < ops.size(); ++i) {
        float p = ops[i].param;
        // Dropout in a fused group scales by 1/(1-rate) computed in f32
        // (lazy.rs:1795-1803).
        if (ops[i].opcode == CLOVE_OP_DROPOUT) p = 1.0f / (1.0f - ops[i].param);
        args.param[i] = p;
    }
    args.numel = numel;
    args.nvec = aligned ? numel / 4 : 0;

    const std::string sig = signature(ops, modes, wide);
    auto it = g_cache.find(sig);
    if (it == g_cache.end()) {
        const std::string name = kernel_name(ops, modes);
        Compiled comp = compile(
            generate(ops, modes, wide, nstore, name, chain_unroll(), chain_block()), name);
        it = g_cache.emplace(sig, comp).first;
    }

    // Grid: enough blocks to cover the vectors once at the chain's unroll,
    // capped at a number of blocks per CU (a grid-stride loop covers the
    // rest).
    const uint64_t threads = (uint64_t)chain_block();
    const uint64_t per_block = threads * chain_unroll();
    uint64_t blocks = (args.nvec + per_block - 1) / per_block;
    if (blocks == 0) blocks = (numel + threads - 1) / threads;
    const uint64_t cap = (uint64_t)c.num_cus * chain_blocks_per_cu();
    if (blocks > cap) blocks = cap;
    if (blocks == 0) blocks = 1;
    void *params[] = {&args};
    CLOVE_HIP_CHECK(hipModuleLaunchKernel(it->second.fn, (unsigned)blocks, 1, 1, (unsigned)threads,
                                          1, 1, 0,
                                          c.stream, params, nullptr));
}

void jit_shutdown() {
    for (auto &kv : g_cache) (void)hipModuleUnload(kv.second.module);
    g_cache.clear();
}

int jit_compiled_count() { return (int)g_cache.size(); }

void jit_stats(int *compiled, int *disk_loads) {
    if (compiled) *compiled = g_compiles;
    if (disk_loads) *disk_loads = g_disk_loads;
}

}  // namespace clove
