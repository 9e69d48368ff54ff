// attention.cpp -- host side of the attention prefill and of RoPE: shape
// rules, the RoPE frequency table, and the launches (kernels/flash_attention.hip).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <map>

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

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// 10000^(i / head_dim) for even i, with the host's f32 powf: the divisor of
// backend.rs:2818 (`abs_pos as f32 / 10000.0f32.powf(i as f32 / head_dim as f32)`).
k::AttnFreq rope_freq(int head_dim) {
    k::AttnFreq f{};
    for (int i = 0; i < head_dim && i / 2 < 128; i += 2)
        f.div[i / 2] = powf(10000.0f, (float)i / (float)head_dim);
    return f;
}

// [B, S, X] (3-d) or [S, X] (2-d, B = 1)
void bsx(const Tensor &t, const char *what, size_t *B, size_t *S, size_t *X) {
    CLOVE_REQUIRE(t.shape.size() == 2 || t.shape.size() == 3, CLOVE_HIP_ERR_SHAPE,
                  std::string(what) + " must be [S, X] or [B, S, X], got " + shape_str(t.shape));
    *B = t.shape.size() == 3 ? t.shape[0] : 1;
    *S = t.shape[t.shape.size() - 2];
    *X = t.shape.back();
}

// One (cos, sin) table per head_dim covering positions [0, npos), built on
// the first call that needs it and regrown (powers of two) when a call needs
// later positions.  Every entry is a function of (position, pair, head_dim)
// alone, so a cached table holds the same bits as a table built for the call.
// It is rebuilt when the library's stream changes, so it is only ever read by
// work enqueued after it on the stream that wrote it.  API calls hold the
// API mutex, which also guards this map.
struct RopeCache {
    TensorNode tab;
    int npos = 0;
    hipStream_t stream = nullptr;
};
std::map<int, RopeCache> g_rope_cache;
constexpr int64_t kRopeCacheMaxFloats = 16 << 20;  // 64 MiB per head_dim at most

}  // namespace

void rope_cache_clear() { g_rope_cache.clear(); }

// A (cos, sin) table whose rows cover positions [pos0, pos0 + npos) for
// head_dim; *tab_pos0 receives the position of the table's first row.
TensorNode rope_table_for(int pos0, int npos, int head_dim, int *tab_pos0) {
    hipStream_t s = ctx().stream;
    const int64_t end = (int64_t)pos0 + npos;
    int64_t n = 1024;
    while (n < end) n *= 2;
    if (n * head_dim <= kRopeCacheMaxFloats) {
        RopeCache &c = g_rope_cache[head_dim];
        if (c.tab == nullptr || c.npos < end || c.stream != s) {
            if (c.npos > n) n = c.npos;
            c.tab = new_tensor({(size_t)n * (size_t)head_dim}, CLOVE_HIP_F32);
            k::rope_table(c.tab->f32(), 0, (int)n, head_dim, rope_freq(head_dim), s);
            c.npos = (int)n;
            c.stream = s;
        }
        *tab_pos0 = 0;
        return c.tab;
    }
    TensorNode tab = new_tensor({(size_t)npos * (size_t)head_dim}, CLOVE_HIP_F32);
    k::rope_table(tab->f32(), pos0, npos, head_dim, rope_freq(head_dim), s);
    *tab_pos0 = pos0;
    return tab;
}

// lazy.rs:1621-1690 (the FlashAttention pattern) and :4821-4909 (its
// kernel): q [B, S, H*D], k and v [B, Sk, H*D].  flags: causal mask and
// RoPE on q and k (k in one pass before the kernel, q inside it) at
// positions s + q_pos and t + k_pos.  The mask hides key t from query s when
// t + mask_k > s + mask_q: the eager entry masks on absolute positions
// (mask_q = q_pos, mask_k = k_pos); the planner's fused step masks on row
// indices as the reference kernel does (lazy.rs:4882: key_idx > row).
// scale <= 0 means 1/sqrt(D), the reference's.
void HipBackend::flash_attention_into(const Tensor &q, const Tensor &k, const Tensor &v,
                                      int num_heads, int q_pos, int k_pos, int mask_q,
                                      int mask_k, int flags, float scale, Tensor &out) {
    CLOVE_REQUIRE(q.dtype == CLOVE_HIP_F32 && k.dtype == CLOVE_HIP_F32 &&
                      v.dtype == CLOVE_HIP_F32 && out.dtype == CLOVE_HIP_F32,
                  CLOVE_HIP_ERR_INVALID, "flash_attention: q, k, v must be f32 tensors");
    size_t B, S, X, Bk, Sk, Xk, Bv, Sv, Xv;
    bsx(q, "q", &B, &S, &X);
    bsx(k, "k", &Bk, &Sk, &Xk);
    bsx(v, "v", &Bv, &Sv, &Xv);
    CLOVE_REQUIRE(Bk == B && Bv == B && Xk == X && Xv == X && Sv == Sk, CLOVE_HIP_ERR_SHAPE,
                  "flash_attention: q " + shape_str(q.shape) + ", k " + shape_str(k.shape) +
                      ", v " + shape_str(v.shape) + " do not agree");
    CLOVE_REQUIRE(num_heads >= 1 && X % (size_t)num_heads == 0, CLOVE_HIP_ERR_SHAPE,
                  "flash_attention: num_heads must divide the last dimension");
    const int D = (int)(X / (size_t)num_heads);
    CLOVE_REQUIRE(k::attention_supported(D), CLOVE_HIP_ERR_SHAPE,
                  "flash_attention: head_dim " + std::to_string(D) + " (1.." +
                      std::to_string(k::kAttnMaxHeadDim) + " have kernels)");
    CLOVE_REQUIRE(!(flags & CLOVE_ATTN_ROPE) || D % 2 == 0, CLOVE_HIP_ERR_SHAPE,
                  "flash_attention: RoPE needs an even head_dim");
    CLOVE_REQUIRE((flags & ~(CLOVE_ATTN_CAUSAL | CLOVE_ATTN_ROPE)) == 0, CLOVE_HIP_ERR_INVALID,
                  "flash_attention: unknown flag");
    CLOVE_REQUIRE(q_pos >= 0 && k_pos >= 0 && mask_q >= 0 && mask_k >= 0,
                  CLOVE_HIP_ERR_INVALID, "flash_attention: positions must be >= 0");
    CLOVE_REQUIRE(B * S < (1ull << 31) && B * Sk < (1ull << 31) &&
                      (size_t)q_pos + S < (1ull << 30) && (size_t)k_pos + Sk < (1ull << 30) &&
                      (size_t)mask_q + S < (1ull << 30) && (size_t)mask_k + Sk < (1ull << 30),
                  CLOVE_HIP_ERR_SHAPE, "flash_attention: too many tokens");
    // the kernel addresses one batch's K or V rows with 32-bit byte offsets
    CLOVE_REQUIRE(Sk * X * 4 < (1ull << 31), CLOVE_HIP_ERR_SHAPE,
                  "flash_attention: one batch's k or v exceeds 2 GiB");
    // one 256-thread workgroup per (batch, head, block of 128 queries)
    CLOVE_REQUIRE(B * (size_t)num_heads * ((S + 127) / 128) * 256 < (1ull << 32),
                  CLOVE_HIP_ERR_SHAPE, "flash_attention: too many query blocks for one grid");
    CLOVE_REQUIRE(out.numel >= q.numel, CLOVE_HIP_ERR_SHAPE, "flash_attention: output too small");
    // 16-byte pieces when D % 4 == 0 (every row then starts 16-byte aligned),
    // single floats otherwise
    const bool vec4 = D % 4 == 0;
    CLOVE_REQUIRE(!vec4 || (aligned16(q.data) && aligned16(k.data) && aligned16(v.data) &&
                            aligned16(out.data)),
                  CLOVE_HIP_ERR_INVALID, "flash_attention: q, k, v must be 16-byte aligned");
    if (q.numel == 0) return;
    const float sc = scale > 0.0f ? scale : 1.0f / sqrtf((float)D);
    hipStream_t s = ctx().stream;
    const float *kp = k.f32(), *qp = q.f32();
    TensorNode kr, qr, tab;
    int t0 = 0;
    if (flags & CLOVE_ATTN_ROPE) {
        // k is rotated in one pass (every query block stages the same keys);
        // q is rotated inside the kernel, once per query, from the same table
        // (in a pass of its own too when rows move as single floats)
        const int p0 = std::min(q_pos, k_pos);
        const int p1 = (int)std::max((size_t)q_pos + S, (size_t)k_pos + Sk);
        tab = rope_table_for(p0, p1 - p0, D, &t0);
        kr = new_tensor(k.shape, CLOVE_HIP_F32);
        k::rope_apply(kp, kr->f32(), B * Sk, (int)Sk, (int)X, D, k_pos, tab->f32(), t0, s);
        kp = kr->f32();
        if (!vec4) {
            qr = new_tensor(q.shape, CLOVE_HIP_F32);
            k::rope_apply(qp, qr->f32(), B * S, (int)S, (int)X, D, q_pos, tab->f32(), t0, s);
            qp = qr->f32();
        }
    }
    // The kernel reads query s's table row at s + (its q_pos) - (its
    // tab_pos0); passing the mask offset as its q_pos and shifting the table
    // origin by the difference keeps that row at s + q_pos.
    const bool q_tab = tab != nullptr && vec4;
    k::attention_prefill(qp, kp, v.f32(), out.f32(), (int)B, (int)S, (int)Sk, num_heads, D,
                         mask_q, mask_k, (flags & CLOVE_ATTN_CAUSAL) != 0, sc,
                         q_tab ? tab->f32() : nullptr, t0 - (q_pos - mask_q), s);
}

TensorNode HipBackend::flash_attention(const TensorNode &q_, const TensorNode &k_,
                                       const TensorNode &v_, int num_heads, int q_pos, int k_pos,
                                       int flags, float scale) {
    const Tensor &q = need(q_, "q");
    const Tensor &k = need(k_, "k");
    const Tensor &v = need(v_, "v");
    TensorNode out = new_tensor(q.shape, CLOVE_HIP_F32);
    flash_attention_into(q, k, v, num_heads, q_pos, k_pos, q_pos, k_pos, flags, scale, *out);
    return out;
}

// backend.rs:2797-2826: x [B, S, hidden] or [S, hidden].
void HipBackend::rope_into(const Tensor &x, size_t pos_offset, size_t head_dim, Tensor &out) {
    CLOVE_REQUIRE(x.dtype == CLOVE_HIP_F32 && out.dtype == CLOVE_HIP_F32, CLOVE_HIP_ERR_INVALID,
                  "rope: x must be an f32 tensor");
    size_t B, S, X;
    bsx(x, "x", &B, &S, &X);
    CLOVE_REQUIRE(head_dim >= 2 && head_dim % 2 == 0 && head_dim <= 256, CLOVE_HIP_ERR_SHAPE,
                  "rope: head_dim must be even and at most 256");
    CLOVE_REQUIRE(X % 2 == 0, CLOVE_HIP_ERR_SHAPE, "rope: the hidden size must be even");
    CLOVE_REQUIRE(pos_offset + S < (1ull << 30) && X < (1ull << 31), CLOVE_HIP_ERR_SHAPE,
                  "rope: positions or hidden size exceed 2^30");
    CLOVE_REQUIRE(out.numel >= x.numel, CLOVE_HIP_ERR_SHAPE, "rope: output too small");
    if (x.numel == 0) return;
    int t0 = 0;
    TensorNode tab = rope_table_for((int)pos_offset, (int)S, (int)head_dim, &t0);
    k::rope_apply(x.f32(), out.f32(), B * S, (int)S, (int)X, (int)head_dim, (int)pos_offset,
                  tab->f32(), t0, ctx().stream);
}

TensorNode HipBackend::rope(const TensorNode &x_, size_t pos_offset, size_t head_dim) {
    const Tensor &x = need(x_, "x");
    TensorNode out = new_tensor(x.shape, CLOVE_HIP_F32);
    rope_into(x, pos_offset, head_dim, *out);
    return out;
}

}  // namespace clove
