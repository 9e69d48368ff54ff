// grad.cpp -- the backward passes and losses of the hot path: the autograd
// closures Clove attaches to matmul, add/sub, relu, gelu and softmax, and
// its cross-entropy and MSE losses (backend.rs), lowered to gfx950 kernels.
//
// Elementwise backward ops run as one-op fused chains (the same device code
// the planner emits for ReluGrad / GeluGrad, lazy.rs:1757-1779); the rest
// use the row kernels (rowwise.hip), the deterministic reductions
// (reduce.hip) and the MFMA GEMM.  Nothing here synchronises.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdlib>

#include "common.hpp"
#include "kernels/launch.hpp"
#include "runtime.hpp"

namespace clove {

namespace {

const Tensor &need(const TensorNode &t, const char *what) {
    CLOVE_REQUIRE(t != nullptr, CLOVE_HIP_ERR_INVALID, std::string(what) + " is NULL");
    CLOVE_REQUIRE(t->dtype == CLOVE_HIP_F32, CLOVE_HIP_ERR_INVALID,
                  std::string(what) + " must be an f32 tensor");
    return *t;
}

// A non-owning 2-d view of t as [rows, cols].
void view2d(const Tensor &t, size_t rows, size_t cols, Tensor *v) {
    v->data = t.data;
    v->shape = {rows, cols};
    v->dtype = t.dtype;
    v->numel = rows * cols;
    v->bytes = t.bytes;
    v->owned = false;
}

void rows_cols(const Tensor &a, size_t *rows, size_t *cols) {
    CLOVE_REQUIRE(!a.shape.empty(), CLOVE_HIP_ERR_SHAPE, "row op needs at least 1 dimension");
    *cols = a.shape.back();
    *rows = *cols ? a.numel / *cols : 0;
    CLOVE_REQUIRE(*rows < (1ull << 31) && *cols < (1ull << 31), CLOVE_HIP_ERR_SHAPE,
                  "row op dimensions exceed 2^31");
}

TensorNode elementwise_grad(int opcode, const TensorNode &x_, const TensorNode &g_) {
    const Tensor &x = need(x_, "x");
    const Tensor &g = need(g_, "grad_out");
    CLOVE_REQUIRE(x.numel == g.numel, CLOVE_HIP_ERR_SHAPE,
                  "grad_out " + shape_str(g.shape) + " does not match x " + shape_str(x.shape));
    TensorNode out = new_tensor(x.shape, CLOVE_HIP_F32);
    if (x.numel == 0) return out;
    ChainOp op;
    op.opcode = opcode;
    op.src0 = -1;
    op.src1 = -2;
    run_chain({op}, {&x, &g}, {out.get()}, x.numel);
    return out;
}

}  // namespace

// backend.rs:1858-1870: the parent's gradient is grad_out where relu's
// output is positive, which is where x is positive.
TensorNode HipBackend::relu_backward(const TensorNode &x, const TensorNode &grad_out) {
    return elementwise_grad(CLOVE_OP_RELU_GRAD, x, grad_out);
}

// backend.rs:1965-1981.
TensorNode HipBackend::gelu_backward(const TensorNode &x, const TensorNode &grad_out) {
    return elementwise_grad(CLOVE_OP_GELU_GRAD, x, grad_out);
}

// backend.rs:2163-2183: rows of y = softmax(x) and of grad_out.
TensorNode HipBackend::softmax_backward(const TensorNode &y_, const TensorNode &g_) {
    const Tensor &y = need(y_, "y");
    const Tensor &g = need(g_, "grad_out");
    CLOVE_REQUIRE(y.numel == g.numel && !y.shape.empty() && !g.shape.empty() &&
                      y.shape.back() == g.shape.back(),
                  CLOVE_HIP_ERR_SHAPE,
                  "grad_out " + shape_str(g.shape) + " does not match y " + shape_str(y.shape));
    size_t rows, cols;
    rows_cols(y, &rows, &cols);
    TensorNode out = new_tensor(y.shape, CLOVE_HIP_F32);
    k::softmax_backward_rows(y.f32(), g.f32(), out->f32(), rows, cols, ctx().stream);
    return out;
}

// backend.rs:1314-1360: grad_a = grad_out . b^T (a's shape, m = prod of a's
// leading dims), grad_b = a^T . grad_out ([k, n]).  Each product is the MFMA
// GEMM; where its plan allows (128x128, 128x256 and 64x128 tilings, split
// over K or not, whose operand rows hold whole 16-byte pieces) the GEMM reads
// the transposed operand directly (k::gemm_f32_transposed), else it runs on a
// transposed copy with the same plan.  Both give the same bits.
// CLOVE_GEMM_TRANSPOSED=0 forces the copies (tests).
static bool transposed_loads_enabled() {
    const char *v = std::getenv("CLOVE_GEMM_TRANSPOSED");
    return !(v && v[0] == '0');
}

void HipBackend::matmul_backward(const TensorNode &a_, const TensorNode &b_, const TensorNode &g_,
                                 TensorNode *grad_a, TensorNode *grad_b) {
    const Tensor &a = need(a_, "a");
    const Tensor &b = need(b_, "b");
    const Tensor &g = need(g_, "grad_out");
    CLOVE_REQUIRE(!a.shape.empty() && b.shape.size() == 2, CLOVE_HIP_ERR_SHAPE,
                  "matmul_backward: a needs >= 1 dimension and b exactly 2");
    const size_t kk = a.shape.back();
    const size_t m = kk ? a.numel / kk : 0;
    const size_t n = b.shape[1];
    CLOVE_REQUIRE(b.shape[0] == kk, CLOVE_HIP_ERR_SHAPE,
                  "matmul_backward: inner dimensions differ, a " + shape_str(a.shape) + " b " +
                      shape_str(b.shape));
    CLOVE_REQUIRE(g.numel == m * n, CLOVE_HIP_ERR_SHAPE,
                  "matmul_backward: grad_out " + shape_str(g.shape) + " is not " +
                      std::to_string(m) + " x " + std::to_string(n));
    CLOVE_REQUIRE(m < (1ull << 31) && n < (1ull << 31) && kk < (1ull << 31), CLOVE_HIP_ERR_SHAPE,
                  "matmul dimensions exceed 2^31");
    hipStream_t s = ctx().stream;
    Tensor gv;
    view2d(g, m, n, &gv);
    const bool direct = transposed_loads_enabled();
    const int cus = ctx().num_cus;
    if (grad_a) {  // [m, n] . ([kk, n])^T
        TensorNode da = new_tensor(a.shape, CLOVE_HIP_F32);
        Tensor dav;
        view2d(*da, m, kk, &dav);
        const k::GemmPlan p = k::gemm_plan((int)m, (int)kk, (int)n, cus, -1);
        TensorNode ws;
        if (direct && p.ws_floats) ws = new_tensor({p.ws_floats}, CLOVE_HIP_F32);
        if (!(direct && k::gemm_f32_transposed(p, g.f32(), b.f32(), da->f32(),
                                               ws ? ws->f32() : nullptr, false, true, s))) {
            TensorNode bt = new_tensor({n, kk}, CLOVE_HIP_F32);
            k::transpose(b.f32(), bt->f32(), kk, n, s);
            matmul_into(gv, *bt, dav);
        }
        *grad_a = da;
    }
    if (grad_b) {  // ([m, kk])^T . [m, n]
        TensorNode db = new_tensor({kk, n}, CLOVE_HIP_F32);
        const k::GemmPlan p = k::gemm_plan((int)kk, (int)n, (int)m, cus, -1);
        TensorNode ws;
        if (direct && p.ws_floats) ws = new_tensor({p.ws_floats}, CLOVE_HIP_F32);
        if (!(direct && k::gemm_f32_transposed(p, a.f32(), g.f32(), db->f32(),
                                               ws ? ws->f32() : nullptr, true, false, s))) {
            TensorNode at = new_tensor({kk, m}, CLOVE_HIP_F32);
            k::transpose(a.f32(), at->f32(), m, kk, s);
            matmul_into(*at, gv, *db);
        }
        *grad_b = db;
    }
}

// backend.rs:1527-1538 (add) and 1800-1810 (sub): the broadcast operand's
// gradient, gb[i % b_numel] (+/-)= grad_out[i], summed without atomics.
TensorNode HipBackend::broadcast_grad(const TensorNode &g_, size_t b_numel, bool negate) {
    const Tensor &g = need(g_, "grad_out");
    CLOVE_REQUIRE(b_numel > 0, CLOVE_HIP_ERR_SHAPE, "broadcast_grad: b has no elements");
    TensorNode out = new_tensor({b_numel}, CLOVE_HIP_F32);
    TensorNode ws =
        new_tensor({std::max<size_t>(k::broadcast_grad_workspace(g.numel, b_numel), 1)},
                   CLOVE_HIP_F32);
    k::broadcast_grad(g.f32(), g.numel, b_numel, negate, ws->f32(), out->f32(), ctx().stream);
    return out;
}

// backend.rs:2661-2680: logits [rows, cols] (rows = all leading dims),
// targets hold f32 class indices; the first min(rows, numel(targets)) rows
// contribute and the sum is divided by rows.  A class >= cols (a panic in
// the reference) is reported at the next synchronising call.
TensorNode HipBackend::cross_entropy(const TensorNode &l_, const TensorNode &t_) {
    const Tensor &l = need(l_, "logits");
    const Tensor &t = need(t_, "targets");
    size_t rows, cols;
    rows_cols(l, &rows, &cols);
    const size_t used = std::min(rows, t.numel);
    TensorNode out = new_tensor({1, 1}, CLOVE_HIP_F32);
    TensorNode rowv = new_tensor({std::max<size_t>(rows, 1)}, CLOVE_HIP_F32);
    hipStream_t s = ctx().stream;
    k::cross_entropy_rows(l.f32(), t.f32(), used, rows, cols, rowv->f32(), device_error_flag(), s);
    k::ordered_sum(rowv->f32(), rows, -1.0f, (float)rows, out->f32(), s);
    return out;
}

// backend.rs:2686-2712: grad_loss is the loss's gradient (one element).
TensorNode HipBackend::cross_entropy_backward(const TensorNode &l_, const TensorNode &t_,
                                              const TensorNode &gl_) {
    const Tensor &l = need(l_, "logits");
    const Tensor &t = need(t_, "targets");
    const Tensor &gl = need(gl_, "grad_loss");
    CLOVE_REQUIRE(gl.numel >= 1, CLOVE_HIP_ERR_SHAPE, "grad_loss is empty");
    size_t rows, cols;
    rows_cols(l, &rows, &cols);
    TensorNode out = new_tensor(l.shape, CLOVE_HIP_F32);
    k::cross_entropy_backward_rows(l.f32(), t.f32(), std::min(rows, t.numel), rows, cols, gl.f32(),
                                   out->f32(), device_error_flag(), ctx().stream);
    return out;
}

// backend.rs:2765-2772: mean of (pred - target)^2 over pred's elements;
// target must have at least as many (the reference indexes it by pred's).
TensorNode HipBackend::mse(const TensorNode &p_, const TensorNode &t_) {
    const Tensor &p = need(p_, "pred");
    const Tensor &t = need(t_, "target");
    CLOVE_REQUIRE(t.numel >= p.numel, CLOVE_HIP_ERR_SHAPE,
                  "target " + shape_str(t.shape) + " is smaller than pred " + shape_str(p.shape));
    TensorNode out = new_tensor({1, 1}, CLOVE_HIP_F32);
    TensorNode ws = new_tensor({std::max<size_t>(k::sq_diff_workspace(p.numel), 1)}, CLOVE_HIP_F32);
    k::mse_loss(p.f32(), t.f32(), p.numel, ws->f32(), out->f32(), ctx().stream);
    return out;
}

// backend.rs:2780-2790.
TensorNode HipBackend::mse_backward(const TensorNode &p_, const TensorNode &t_,
                                    const TensorNode &gl_) {
    const Tensor &p = need(p_, "pred");
    const Tensor &t = need(t_, "target");
    const Tensor &gl = need(gl_, "grad_loss");
    CLOVE_REQUIRE(t.numel >= p.numel, CLOVE_HIP_ERR_SHAPE,
                  "target " + shape_str(t.shape) + " is smaller than pred " + shape_str(p.shape));
    CLOVE_REQUIRE(gl.numel >= 1, CLOVE_HIP_ERR_SHAPE, "grad_loss is empty");
    TensorNode out = new_tensor(p.shape, CLOVE_HIP_F32);
    k::mse_backward(p.f32(), t.f32(), p.numel, gl.f32(), out->f32(), ctx().stream);
    return out;
}

// optim.rs:375-395: every parameter tensor w with its gradient g and
// moments m, v (all f32, same element count) updated in place.  The bias
// corrections 1 - beta^t use the host's powf on (float)step, as the
// reference computes them.
void HipBackend::adamw_step(const std::vector<const Tensor *> &w,
                            const std::vector<const Tensor *> &g,
                            const std::vector<const Tensor *> &m,
                            const std::vector<const Tensor *> &v, const AdamWParams &p) {
    const size_t count = w.size();
    CLOVE_REQUIRE(g.size() == count && m.size() == count && v.size() == count,
                  CLOVE_HIP_ERR_INVALID, "adamw: w, g, m, v lists differ in length");
    CLOVE_REQUIRE(p.step >= 1, CLOVE_HIP_ERR_INVALID,
                  "adamw: step counts from 1 (AdamW::step increments before updating)");
    std::vector<float *> pw(count), pm(count), pv(count);
    std::vector<const float *> pg(count);
    std::vector<uint64_t> n(count);
    for (size_t i = 0; i < count; ++i) {
        const Tensor *t[4] = {w[i], g[i], m[i], v[i]};
        const char *what[4] = {"w", "g", "m", "v"};
        for (int j = 0; j < 4; ++j) {
            CLOVE_REQUIRE(t[j] != nullptr, CLOVE_HIP_ERR_INVALID,
                          std::string("adamw: ") + what[j] + "[" + std::to_string(i) + "] is NULL");
            CLOVE_REQUIRE(t[j]->dtype == CLOVE_HIP_F32, CLOVE_HIP_ERR_INVALID,
                          std::string("adamw: ") + what[j] + " must be f32");
            CLOVE_REQUIRE(t[j]->numel == w[i]->numel, CLOVE_HIP_ERR_SHAPE,
                          "adamw: tensor " + std::to_string(i) + " has mismatched sizes");
        }
        pw[i] = w[i]->f32();
        pg[i] = g[i]->f32();
        pm[i] = m[i]->f32();
        pv[i] = v[i]->f32();
        n[i] = w[i]->numel;
    }
    const float t = (float)p.step;
    const k::AdamWHyper h{p.lr, p.beta1, p.beta2, p.eps, p.weight_decay, p.loss_scale, p.clip,
                          1.0f - powf(p.beta1, t), 1.0f - powf(p.beta2, t)};
    Context &c = ctx();
    k::adamw_step(pw.data(), pg.data(), pm.data(), pv.data(), n.data(), (int)count, h, c.num_cus,
                  c.stream);
}

}  // namespace clove
