// ops.cpp -- the eager HIP backend: the hot-path methods of Clove's
// `trait Backend` (backend.rs:171-257) with the shape rules of WgpuBackend,
// lowered to the gfx950 kernels.  Every op allocates its output through the
// caching allocator and enqueues its kernels on the context stream; nothing
// here synchronises.
//
// Elementwise ops run as one-op fused chains (jit.cpp), the same kernels the
// lazy planner emits for longer chains, so eager and fused results are
// produced by identical device code.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>

#include "common.hpp"
#include "kernels/launch.hpp"
#include "runtime.hpp"

namespace clove {

namespace {

const Tensor &need(const TensorNode &t, const char *what) {
    CLOVE_REQUIRE(t != nullptr, CLOVE_HIP_ERR_INVALID, std::string(what) + " is NULL");
    return *t;
}

void need_f32(const Tensor &t, const char *what) {
    CLOVE_REQUIRE(t.dtype == CLOVE_HIP_F32, CLOVE_HIP_ERR_INVALID,
                  std::string(what) + " must be an f32 tensor");
}

// The int32 views of a block table and a context-length tensor.  Clove
// builds every tensor from a Vec<f32> (backend.rs:176, ffi.rs:71-87), so its
// paged_attention receives both as f32 tensors (backend.rs:249-256,
// nn.rs:528-546); int32 tensors are used as they are.  f32 ones are
// converted on the device into temporaries, in one launch: an integer value
// in [0, 2^24) is taken as is, anything else becomes -1 and, for a context
// length or a table entry the context reaches, is reported as
// CLOVE_HIP_ERR_RANGE by the next synchronising call (a -1 entry lies outside
// the pool and its tokens are skipped; a -1 context length counts as 0).
// Entries past a sequence's blocks are never read, so their values do not
// matter, as with int32 tables.
struct IndexPair {
    const int32_t *bt = nullptr, *cl = nullptr;
    TensorNode bt_tmp, cl_tmp;
};

IndexPair index_pair(const Tensor &bt, const Tensor &cl, int block_size) {
    auto ok = [](const Tensor &t) { return t.dtype == CLOVE_HIP_I32 || t.dtype == CLOVE_HIP_F32; };
    CLOVE_REQUIRE(ok(bt) && ok(cl), CLOVE_HIP_ERR_INVALID,
                  "block_tables and context_lens must be int32 or f32 tensors");
    CLOVE_REQUIRE(bt.shape.size() == 2 && bt.shape[0] == cl.numel && bt.shape[1] < (1ull << 31),
                  CLOVE_HIP_ERR_SHAPE,
                  "block_tables must be [num_seqs, max_blocks] with num_seqs = numel(context_lens)");
    IndexPair p;
    if (bt.dtype == CLOVE_HIP_F32) p.bt_tmp = new_tensor(bt.shape, CLOVE_HIP_I32);
    if (cl.dtype == CLOVE_HIP_F32) p.cl_tmp = new_tensor(cl.shape, CLOVE_HIP_I32);
    if (p.bt_tmp || p.cl_tmp)
        k::paged_index_from_f32(p.bt_tmp ? bt.f32() : nullptr, p.bt_tmp ? p.bt_tmp->i32() : nullptr,
                                p.cl_tmp ? cl.f32() : nullptr, p.cl_tmp ? nullptr : cl.i32(),
                                p.cl_tmp ? p.cl_tmp->i32() : nullptr, (int)cl.numel,
                                (int)bt.shape[1], block_size, device_error_flag(), ctx().stream);
    p.bt = p.bt_tmp ? p.bt_tmp->i32() : bt.i32();
    p.cl = p.cl_tmp ? p.cl_tmp->i32() : cl.i32();
    return p;
}

}  // namespace

TensorNode HipBackend::new_cpu(const float *data, const std::vector<size_t> &shape) {
    TensorNode t = new_tensor(shape, CLOVE_HIP_F32);
    if (data) upload(*t, data, 0, t->numel);
    return t;
}

// backend.rs:1483-1493 (add), :1748-1758 (sub), :1598-1617 (mul): the output
// has a's shape and b is read as b[i % numel(b)].
TensorNode HipBackend::binary(int opcode, const TensorNode &a_, const TensorNode &b_) {
    const Tensor &a = need(a_, "a");
    const Tensor &b = need(b_, "b");
    need_f32(a, "a");
    need_f32(b, "b");
    CLOVE_REQUIRE(b.numel > 0 || a.numel == 0, CLOVE_HIP_ERR_SHAPE,
                  "broadcast operand b is empty");
    TensorNode out = new_tensor(a.shape, CLOVE_HIP_F32);
    if (a.numel == 0) return out;
    ChainOp op;
    op.opcode = opcode;
    op.src0 = -1;
    op.src1 = -2;
    run_chain({op}, {&a, &b}, {out.get()}, a.numel);
    return out;
}

TensorNode HipBackend::unary(int opcode, const TensorNode &a_, float param) {
    const Tensor &a = need(a_, "a");
    need_f32(a, "a");
    TensorNode out = new_tensor(a.shape, CLOVE_HIP_F32);
    if (a.numel == 0) return out;
    ChainOp op;
    op.opcode = opcode;
    op.src0 = -1;
    op.param = param;
    run_chain({op}, {&a}, {out.get()}, a.numel);
    return out;
}

// backend.rs:2266-2336: the 2-d transpose [rows, cols] -> [cols, rows] (the
// LDS-tiled transpose the matmul backward uses; a pure permutation, so the
// same bits as the reference's loop).
TensorNode HipBackend::transpose(const TensorNode &a_) {
    const Tensor &a = need(a_, "a");
    need_f32(a, "a");
    CLOVE_REQUIRE(a.shape.size() == 2, CLOVE_HIP_ERR_SHAPE,
                  "transpose: a must be 2-d, got " + shape_str(a.shape));
    const size_t rows = a.shape[0], cols = a.shape[1];
    TensorNode out = new_tensor({cols, rows}, CLOVE_HIP_F32);
    if (a.numel) k::transpose(a.f32(), out->f32(), rows, cols, ctx().stream);
    return out;
}

// backend.rs:2337-2370: a copy of a with shape [1, numel] (the fused chain's
// Flatten copy, 16-byte streaming loads and stores).
TensorNode HipBackend::flatten(const TensorNode &a_) {
    TensorNode out = unary(CLOVE_OP_FLATTEN, a_);
    out->shape = {1, out->numel};
    return out;
}

// backend.rs:1437-1482: per batch, a's s1 rows and then b's s2 rows of h
// floats; a 2-d operand is one batch, and the result has a's rank ([B, s1 +
// s2, h] or [s1 + s2, h]).  The reference builds it on the host; here two
// strided device copies.
TensorNode HipBackend::concat_seq(const TensorNode &a_, const TensorNode &b_) {
    const Tensor &a = need(a_, "a");
    const Tensor &b = need(b_, "b");
    need_f32(a, "a");
    need_f32(b, "b");
    auto bsh = [](const Tensor &t, size_t *B, size_t *S, size_t *H) {
        const size_t r = t.shape.size();
        CLOVE_REQUIRE(r == 2 || r == 3, CLOVE_HIP_ERR_SHAPE,
                      "concat_seq: operands must be 2-d or 3-d, got " + shape_str(t.shape));
        *B = r == 3 ? t.shape[0] : 1;
        *S = t.shape[r - 2];
        *H = t.shape[r - 1];
    };
    size_t B, s1, h, Bb, s2, hb;
    bsh(a, &B, &s1, &h);
    bsh(b, &Bb, &s2, &hb);
    CLOVE_REQUIRE(Bb == B && hb == h, CLOVE_HIP_ERR_SHAPE,
                  "concat_seq: batch and hidden sizes differ, a " + shape_str(a.shape) + " b " +
                      shape_str(b.shape));
    TensorNode out = new_tensor(a.shape.size() == 3 ? std::vector<size_t>{B, s1 + s2, h}
                                                    : std::vector<size_t>{s1 + s2, h},
                                CLOVE_HIP_F32);
    hipStream_t s = ctx().stream;
    const size_t pitch = (s1 + s2) * h * 4, wa = s1 * h * 4, wb = s2 * h * 4;
    if (B && wa)
        CLOVE_HIP_CHECK(hipMemcpy2DAsync(out->data, pitch, a.data, wa, wa, B,
                                         hipMemcpyDeviceToDevice, s));
    if (B && wb)
        CLOVE_HIP_CHECK(hipMemcpy2DAsync(static_cast<char *>(out->data) + wa, pitch, b.data, wb,
                                         wb, B, hipMemcpyDeviceToDevice, s));
    return out;
}

TensorNode HipBackend::add(const TensorNode &a, const TensorNode &b) { return binary(CLOVE_OP_ADD, a, b); }
TensorNode HipBackend::sub(const TensorNode &a, const TensorNode &b) { return binary(CLOVE_OP_SUB, a, b); }
TensorNode HipBackend::mul(const TensorNode &a, const TensorNode &b) { return binary(CLOVE_OP_MUL, a, b); }
TensorNode HipBackend::mul_scalar(const TensorNode &a, float s) { return unary(CLOVE_OP_SCALAR_MUL, a, s); }
TensorNode HipBackend::relu(const TensorNode &a) { return unary(CLOVE_OP_RELU, a); }
TensorNode HipBackend::gelu(const TensorNode &a) { return unary(CLOVE_OP_GELU, a); }
TensorNode HipBackend::sigmoid(const TensorNode &a) { return unary(CLOVE_OP_SIGMOID, a); }
TensorNode HipBackend::tanh(const TensorNode &a) { return unary(CLOVE_OP_TANH, a); }
TensorNode HipBackend::sin(const TensorNode &a) { return unary(CLOVE_OP_SIN, a); }
TensorNode HipBackend::cos(const TensorNode &a) { return unary(CLOVE_OP_COS, a); }

// ---- row reductions --------------------------------------------------------

static void row_dims(const Tensor &a, size_t *rows, size_t *cols) {
    CLOVE_REQUIRE(!a.shape.empty(), CLOVE_HIP_ERR_SHAPE, "row op needs at least 1 dimension");
    *cols = a.shape.back();
    *rows = *cols ? a.numel / *cols : 0;
    CLOVE_REQUIRE(*rows < (1ull << 31) && *cols < (1ull << 31), CLOVE_HIP_ERR_SHAPE,
                  "row op dimensions exceed 2^31");
}

void HipBackend::softmax_into(const Tensor &a, Tensor &out) {
    need_f32(a, "a");
    size_t rows, cols;
    row_dims(a, &rows, &cols);
    k::softmax_rows(a.f32(), out.f32(), rows, cols, ctx().stream);
}

// backend.rs:2102-2125: rows = shape[0], cols = shape[1]; here the last
// dimension is the row, which is the same thing for the 2-d tensors Clove
// passes and extends it to N-d.
TensorNode HipBackend::softmax(const TensorNode &a_) {
    const Tensor &a = need(a_, "a");
    TensorNode out = new_tensor(a.shape, CLOVE_HIP_F32);
    softmax_into(a, *out);
    return out;
}

void HipBackend::layer_norm_into(const Tensor &a, const Tensor &g, const Tensor &b, Tensor &out) {
    need_f32(a, "a");
    need_f32(g, "gamma");
    need_f32(b, "beta");
    size_t rows, cols;
    row_dims(a, &rows, &cols);
    // backend.rs:2401-2403 indexes gamma[j] and beta[j] for j < cols.
    CLOVE_REQUIRE(g.numel >= cols && b.numel >= cols, CLOVE_HIP_ERR_SHAPE,
                  "gamma/beta need at least " + std::to_string(cols) + " elements");
    k::layer_norm_rows(a.f32(), g.f32(), b.f32(), out.f32(), rows, cols, 1e-5f, ctx().stream);
}

TensorNode HipBackend::layer_norm(const TensorNode &a_, const TensorNode &g_, const TensorNode &b_) {
    const Tensor &a = need(a_, "a");
    TensorNode out = new_tensor(a.shape, CLOVE_HIP_F32);
    layer_norm_into(a, need(g_, "gamma"), need(b_, "beta"), *out);
    return out;
}

// ---- matmul ------------------------------------------------------------------

static void matmul_dims(const Tensor &a, const Tensor &b, size_t *m, size_t *k, size_t *n) {
    CLOVE_REQUIRE(!a.shape.empty(), CLOVE_HIP_ERR_SHAPE, "matmul: a needs at least 1 dimension");
    CLOVE_REQUIRE(b.shape.size() == 2, CLOVE_HIP_ERR_SHAPE,
                  "matmul: b must be 2-d, got " + shape_str(b.shape));
    *k = a.shape.back();
    *m = 1;
    for (size_t i = 0; i + 1 < a.shape.size(); ++i) *m *= a.shape[i];
    *n = b.shape[1];
    CLOVE_REQUIRE(b.shape[0] == *k, CLOVE_HIP_ERR_SHAPE,
                  "matmul: inner dimensions differ, a " + shape_str(a.shape) + " b " +
                      shape_str(b.shape));
    CLOVE_REQUIRE(*m < (1ull << 31) && *n < (1ull << 31) && *k < (1ull << 31),
                  CLOVE_HIP_ERR_SHAPE, "matmul dimensions exceed 2^31");
}

// CLOVE_GEMM_CFG selects a tile configuration by index and turns the
// skinny path off; CLOVE_GEMM_SKINNY="nb,splits" forces the skinny path where
// it is legal (M <= 64, K % 4 == 0) and sets its column blocks per wave and
// K splits (0 keeps the default); CLOVE_GEMM_STRIP=1 forces the strip path
// where it is legal (M <= 32, even N).  All are for tuning sweeps and tests
// only: every plan computes the same product.
static int gemm_cfg_override() {
    const char *v = std::getenv("CLOVE_GEMM_CFG");
    return (v && *v) ? std::atoi(v) : -1;
}
static bool gemm_strip_override() {
    const char *v = std::getenv("CLOVE_GEMM_STRIP");
    return v && *v && std::atoi(v) != 0;
}
static bool gemm_skinny_override(int *nb, int *splits) {
    *nb = 0;
    *splits = 0;
    const char *v = std::getenv("CLOVE_GEMM_SKINNY");
    if (!v || !*v) return false;
    if (std::sscanf(v, "%d,%d", nb, splits) < 1) *nb = 0;
    return true;
}

// Validates one product and builds its epilogue and plan.
static k::GemmPlan prepare_matmul(const Tensor &a, const Tensor &b, const Tensor *bias, int act,
                                  k::GemmEpilogue *epi) {
    need_f32(a, "a");
    need_f32(b, "b");
    size_t m, kk, n;
    matmul_dims(a, b, &m, &kk, &n);
    if (bias) {
        need_f32(*bias, "bias");
        CLOVE_REQUIRE(bias->numel > 0, CLOVE_HIP_ERR_SHAPE, "bias is empty");
        epi->bias = bias->f32();
        epi->bias_n = bias->numel;
        epi->bias_mode = bias->numel == 1 ? k::GEMM_BIAS_SCALAR
                         : bias->numel == n ? k::GEMM_BIAS_COL
                                            : k::GEMM_BIAS_MOD;
    }
    CLOVE_REQUIRE(act >= k::GEMM_ACT_NONE && act <= k::GEMM_ACT_SOFTMAX, CLOVE_HIP_ERR_INVALID,
                  "unknown GEMM epilogue activation");
    epi->act = act;
    int sk_nb, sk_splits;
    const bool sk_force = gemm_skinny_override(&sk_nb, &sk_splits);
    const bool a_aligned = (reinterpret_cast<uintptr_t>(a.data) & 15) == 0;
    const bool b_aligned = (reinterpret_cast<uintptr_t>(b.data) & 15) == 0;
    return k::gemm_plan((int)m, (int)n, (int)kk, ctx().num_cus, gemm_cfg_override(), a_aligned,
                        sk_force, sk_nb, sk_splits, gemm_strip_override(), b_aligned);
}

// A product the grouped small kernel can take: the small path, and for a
// softmax epilogue whole rows in one 16-column tile.
static bool groupable(const k::GemmPlan &p, int act) {
    return p.small && (act != k::GEMM_ACT_SOFTMAX || p.N <= 16);
}

void HipBackend::matmul_into(const Tensor &a, const Tensor &b, Tensor &out, const Tensor *bias,
                             int act) {
    k::GemmEpilogue epi;
    const k::GemmPlan p = prepare_matmul(a, b, bias, act, &epi);
    hipStream_t s = ctx().stream;
    TensorNode ws;
    if (p.ws_floats) ws = new_tensor({p.ws_floats}, CLOVE_HIP_F32);
    if (act == k::GEMM_ACT_SOFTMAX && !(p.small && p.tiles_n == 1)) {
        // only the small path with one tile column holds whole rows: product
        // and bias into a temporary, then the row softmax into `out`
        epi.act = k::GEMM_ACT_NONE;
        TensorNode tmp = new_tensor(out.shape, CLOVE_HIP_F32);
        k::gemm_f32(p, a.f32(), b.f32(), tmp->f32(), ws ? ws->f32() : nullptr, epi, s);
        softmax_into(*tmp, out);
        return;
    }
    k::gemm_f32(p, a.f32(), b.f32(), out.f32(), ws ? ws->f32() : nullptr, epi, s);
}

// The lazy path's horizontal MatMul group (lazy.rs:2443-2493, executed at
// :3483-3557 as one compute pass with a dispatch per product): independent
// products whose plans take the small path run in ONE grouped launch (up to
// k::kGemmGroupMax per launch); the others run one by one.
void HipBackend::matmul_group_into(const std::vector<GemmMember> &members) {
    std::vector<k::GemmPlan> plans;
    std::vector<const float *> A, B;
    std::vector<float *> C;
    std::vector<k::GemmEpilogue> epis;
    std::vector<const GemmMember *> rest;
    for (const GemmMember &g : members) {
        k::GemmEpilogue epi;
        const k::GemmPlan p = prepare_matmul(*g.a, *g.b, g.bias, g.act, &epi);
        if (!groupable(p, g.act)) {
            rest.push_back(&g);
            continue;
        }
        plans.push_back(p);
        A.push_back(g.a->f32());
        B.push_back(g.b->f32());
        C.push_back(g.out->f32());
        epis.push_back(epi);
    }
    hipStream_t s = ctx().stream;
    for (size_t i = 0; i < plans.size(); i += k::kGemmGroupMax) {
        const int count = (int)std::min<size_t>(k::kGemmGroupMax, plans.size() - i);
        k::gemm_f32_grouped(&plans[i], &A[i], &B[i], &C[i], &epis[i], count, s);
    }
    for (const GemmMember *g : rest) matmul_into(*g->a, *g->b, *g->out, g->bias, g->act);
}

// backend.rs:1282-1306: m = prod(a.shape[..last]), k = a.shape[last],
// n = b.shape[1]; the output keeps a's leading dims with the last set to n.
TensorNode HipBackend::matmul(const TensorNode &a_, const TensorNode &b_) {
    const Tensor &a = need(a_, "a");
    const Tensor &b = need(b_, "b");
    size_t m, kk, n;
    matmul_dims(a, b, &m, &kk, &n);
    std::vector<size_t> shape = a.shape;
    shape.back() = n;
    TensorNode out = new_tensor(shape, CLOVE_HIP_F32);
    matmul_into(a, b, *out);
    return out;
}

// ---- paged attention -----------------------------------------------------------

// Checks the sizes and alignment both decode entries share and fills the
// kernel arguments (without the workspace); *ws receives the workspace floats
// the launch needs (0 when every context fits one partition).
static k::PagedArgs paged_args(const HipBackend::PagedRaw &r, size_t *ws) {
    const int64_t B = r.num_seqs, H = r.num_heads, D = r.head_dim, bs = r.block_size;
    CLOVE_REQUIRE((int64_t)r.max_blocks * bs < (1ll << 31) && r.num_blocks * bs < (1ll << 31),
                  CLOVE_HIP_ERR_SHAPE, "context capacity exceeds 2^31 tokens");
    // grid: (head groups, partitions, sequences)
    CLOVE_REQUIRE(B < 65536, CLOVE_HIP_ERR_SHAPE, "at most 65535 sequences per launch");
    // 16-byte vector loads when head_dim % 4 == 0, 4-byte loads otherwise
    const uintptr_t amask = D % 4 == 0 ? 15 : 3;
    auto aligned = [amask](const void *p) { return (reinterpret_cast<uintptr_t>(p) & amask) == 0; };
    CLOVE_REQUIRE(aligned(r.q) && aligned(r.k_new) && aligned(r.v_new) && aligned(r.kv_cache) &&
                      aligned(r.out),
                  CLOVE_HIP_ERR_INVALID,
                  D % 4 == 0 ? "q, k, v, kv_cache and out must be 16-byte aligned"
                             : "q, k, v, kv_cache and out must be 4-byte aligned");
    k::PagedArgs a{};
    a.q = r.q;
    a.k_new = r.k_new;
    a.v_new = r.v_new;
    a.k_cache = r.kv_cache;
    a.v_cache = r.kv_cache + (size_t)r.num_blocks * bs * H * D;
    a.block_tables = r.block_tables;
    a.context_lens = r.context_lens;
    a.out = r.out;
    a.err_flag = device_error_flag();
    a.num_blocks = r.num_blocks;
    a.num_seqs = (int)B;
    a.num_heads = (int)H;
    a.head_dim = (int)D;
    a.block_size = (int)bs;
    a.max_blocks = r.max_blocks;
    const int cap = (int)(r.max_blocks * bs);
    a.part_tokens = k::paged_part_tokens((int)B, (int)H, cap, (int)bs, ctx().num_cus);
    a.max_parts = std::max(1, (cap + a.part_tokens - 1) / a.part_tokens);
    CLOVE_REQUIRE(a.max_parts < 65536, CLOVE_HIP_ERR_SHAPE, "too many context partitions");
    a.scale = r.scale;
    *ws = k::paged_workspace_floats((int)B, (int)H, (int)D, cap, a.part_tokens);
    return a;
}

void HipBackend::paged_attention_into(const Tensor &q, const Tensor *kn, const Tensor *vn,
                                      const Tensor &kv, const Tensor &bt, const Tensor &cl,
                                      float scale, Tensor &out) {
    need_f32(q, "q");
    need_f32(kv, "kv_cache");
    CLOVE_REQUIRE((bt.dtype == CLOVE_HIP_I32 || bt.dtype == CLOVE_HIP_F32) &&
                      (cl.dtype == CLOVE_HIP_I32 || cl.dtype == CLOVE_HIP_F32),
                  CLOVE_HIP_ERR_INVALID, "block_tables and context_lens must be int32 or f32 tensors");
    CLOVE_REQUIRE(kv.shape.size() == 5 && kv.shape[0] == 2, CLOVE_HIP_ERR_SHAPE,
                  "kv_cache must be [2, num_blocks, block_size, heads, head_dim], got " +
                      shape_str(kv.shape));
    const size_t nb = kv.shape[1], bs = kv.shape[2], H = kv.shape[3], D = kv.shape[4];
    CLOVE_REQUIRE(k::paged_supported((int)std::min<size_t>(D, 1u << 30), (int)bs),
                  CLOVE_HIP_ERR_SHAPE,
                  "paged attention supports head_dim 1.." + std::to_string(k::kPagedMaxHeadDim) +
                      " and block_size >= 1, got " + std::to_string(D) + "/" + std::to_string(bs));
    const size_t B = cl.numel;
    CLOVE_REQUIRE(bt.shape.size() == 2 && bt.shape[0] == B, CLOVE_HIP_ERR_SHAPE,
                  "block_tables must be [num_seqs, max_blocks] with num_seqs = numel(context_lens)");
    const size_t max_blocks = bt.shape[1];
    CLOVE_REQUIRE(q.numel == B * H * D, CLOVE_HIP_ERR_SHAPE,
                  "q must hold num_seqs*heads*head_dim = " + std::to_string(B * H * D) +
                      " elements, got " + std::to_string(q.numel));
    CLOVE_REQUIRE((kn == nullptr) == (vn == nullptr), CLOVE_HIP_ERR_INVALID,
                  "pass both k and v, or neither");
    if (kn) {
        need_f32(*kn, "k");
        need_f32(*vn, "v");
        CLOVE_REQUIRE(kn->numel == q.numel && vn->numel == q.numel, CLOVE_HIP_ERR_SHAPE,
                      "k and v must have q's number of elements");
    }
    CLOVE_REQUIRE(out.numel >= q.numel, CLOVE_HIP_ERR_SHAPE, "output too small");
    if (B == 0) return;
    const IndexPair idx = index_pair(bt, cl, (int)bs);
    size_t ws = 0;
    k::PagedArgs a = paged_args({q.f32(), kn ? kn->f32() : nullptr, vn ? vn->f32() : nullptr,
                                 kv.f32(), (int64_t)nb, (int)bs, (int)H, (int)D, idx.bt,
                                 (int)max_blocks, idx.cl, (int)B, scale, out.f32()},
                                &ws);
    TensorNode work;
    if (ws) {
        work = new_tensor({ws}, CLOVE_HIP_F32);
        a.partials = work->f32();
    }
    k::paged_attention(a, ctx().stream);
    // `work` and the index temporaries return to the allocator here; later
    // users of those blocks are ordered after these kernels on the same stream.
}

// The allocation-free form: the caller's device memory, int32 indices, and
// the partition workspace in this device's static scratch array.  Nothing
// is allocated and nothing needs clearing (every partial the merge reads is
// written by the same launch).  Two calls never overlap: both run on the
// library's current stream, and set_stream waits for the stream it
// replaces; only replays of a captured call on two streams at once would
// share the array concurrently (the caller orders those).
void HipBackend::paged_attention_noalloc(const PagedRaw &r) {
    CLOVE_REQUIRE(r.num_seqs >= 0 && r.num_heads >= 1 && r.max_blocks >= 1 && r.num_blocks >= 1,
                  CLOVE_HIP_ERR_SHAPE,
                  "num_seqs >= 0, num_heads >= 1, max_blocks >= 1 and num_blocks >= 1 are required");
    CLOVE_REQUIRE(k::paged_supported(r.head_dim, r.block_size), CLOVE_HIP_ERR_SHAPE,
                  "paged attention supports head_dim 1.." + std::to_string(k::kPagedMaxHeadDim) +
                      " and block_size >= 1, got " + std::to_string(r.head_dim) + "/" +
                      std::to_string(r.block_size));
    CLOVE_REQUIRE((r.k_new == nullptr) == (r.v_new == nullptr), CLOVE_HIP_ERR_INVALID,
                  "pass both k and v, or neither");
    if (r.num_seqs == 0) return;
    CLOVE_REQUIRE(r.q && r.kv_cache && r.block_tables && r.context_lens && r.out,
                  CLOVE_HIP_ERR_INVALID, "q, kv_cache, block_tables, context_lens and out are required");
    size_t ws = 0;
    k::PagedArgs a = paged_args(r, &ws);
    CLOVE_REQUIRE(ws <= k::kPagedScratchFloats, CLOVE_HIP_ERR_SHAPE,
                  "the decode needs a " + std::to_string(ws * 4) +
                      "-byte partition workspace; the allocation-free entry has " +
                      std::to_string(k::kPagedScratchFloats * 4) + " bytes of scratch");
    if (ws) a.partials = paged_scratch();
    k::paged_attention(a, ctx().stream);
}

TensorNode HipBackend::paged_attention(const TensorNode &q_, const TensorNode &k_,
                                       const TensorNode &v_, const TensorNode &kv_,
                                       const TensorNode &bt_, const TensorNode &cl_, float scale) {
    const Tensor &q = need(q_, "q");
    TensorNode out = new_tensor(q.shape, CLOVE_HIP_F32);
    paged_attention_into(q, k_.get(), v_.get(), need(kv_, "kv_cache"), need(bt_, "block_tables"),
                         need(cl_, "context_lens"), scale, *out);
    return out;
}

TensorNode HipBackend::paged_gather_indices(const TensorNode &bt_, const TensorNode &cl_,
                                            int block_size, int max_ctx) {
    const Tensor &bt = need(bt_, "block_tables");
    const Tensor &cl = need(cl_, "context_lens");
    CLOVE_REQUIRE(bt.shape.size() == 2 && bt.shape[0] == cl.numel, CLOVE_HIP_ERR_SHAPE,
                  "block_tables must be [num_seqs, max_blocks]");
    CLOVE_REQUIRE(block_size > 0 && max_ctx >= 0, CLOVE_HIP_ERR_INVALID,
                  "block_size must be > 0 and max_ctx >= 0");
    CLOVE_REQUIRE(bt.shape[1] * (size_t)block_size < (1ull << 31) &&
                      cl.numel * (size_t)max_ctx < (1ull << 40),
                  CLOVE_HIP_ERR_SHAPE, "gather indices: sizes exceed the index range");
    const size_t B = cl.numel;
    const IndexPair idx = index_pair(bt, cl, block_size);
    TensorNode out = new_tensor({B, (size_t)max_ctx}, CLOVE_HIP_I32);
    k::paged_slots(idx.bt, idx.cl, out->i32(), (int)B, (int)bt.shape[1], block_size, max_ctx,
                   device_error_flag(), ctx().stream);
    return out;
}

// ---- synthetic data -----------------------------------------------------------

void fill_normal(Tensor &t, uint64_t seed, float mean, float stddev) {
    need_f32(t, "tensor");
    k::fill_normal(t.f32(), t.numel, seed, mean, stddev, ctx().stream);
}

void fill_uniform(Tensor &t, uint64_t seed, float lo, float hi) {
    need_f32(t, "tensor");
    k::fill_uniform(t.f32(), t.numel, seed, lo, hi, ctx().stream);
}

}  // namespace clove

namespace clove {

// KV-cache append (the cache write before decode; no counterpart in Clove).
void HipBackend::paged_kv_append(const Tensor &kv, const Tensor &k, const Tensor &v,
                                 const Tensor &bt, const Tensor &cl) {
    need_f32(kv, "kv_cache");
    need_f32(k, "k");
    need_f32(v, "v");
    CLOVE_REQUIRE((bt.dtype == CLOVE_HIP_I32 || bt.dtype == CLOVE_HIP_F32) &&
                      (cl.dtype == CLOVE_HIP_I32 || cl.dtype == CLOVE_HIP_F32),
                  CLOVE_HIP_ERR_INVALID, "block_tables and context_lens must be int32 or f32 tensors");
    CLOVE_REQUIRE(kv.shape.size() == 5 && kv.shape[0] == 2, CLOVE_HIP_ERR_SHAPE,
                  "kv_cache must be [2, num_blocks, block_size, heads, head_dim], got " +
                      shape_str(kv.shape));
    const size_t nb = kv.shape[1], bs = kv.shape[2], H = kv.shape[3], D = kv.shape[4];
    const size_t B = cl.numel, row = H * D;
    CLOVE_REQUIRE(bt.shape.size() == 2 && bt.shape[0] == B, CLOVE_HIP_ERR_SHAPE,
                  "block_tables must be [num_seqs, max_blocks] with num_seqs = numel(context_lens)");
    CLOVE_REQUIRE(k.numel == B * row && v.numel == B * row, CLOVE_HIP_ERR_SHAPE,
                  "k and v must hold num_seqs*heads*head_dim elements");
    CLOVE_REQUIRE(row % 4 == 0 && ((reinterpret_cast<uintptr_t>(k.data) |
                                    reinterpret_cast<uintptr_t>(v.data) |
                                    reinterpret_cast<uintptr_t>(kv.data)) & 15) == 0,
                  CLOVE_HIP_ERR_INVALID, "kv append needs 16-byte aligned rows");
    CLOVE_REQUIRE(bt.shape[1] * bs < (1ull << 31), CLOVE_HIP_ERR_SHAPE,
                  "context capacity exceeds 2^31 tokens");
    if (B == 0) return;
    const IndexPair idx = index_pair(bt, cl, (int)bs);
    k::paged_append(kv.f32(), kv.f32() + nb * bs * row, k.f32(), v.f32(), idx.bt, idx.cl,
                    (int)B, (int)bt.shape[1], (int)bs, (int64_t)nb, (int)row, device_error_flag(),
                    ctx().stream);
}

}  // namespace clove
