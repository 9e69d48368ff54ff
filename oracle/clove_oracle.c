/*
 * clove_oracle.c -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.
 *
 * A CPU restatement of Clove's Rayon kernels (the eager CPU branch of
 * `WgpuBackend`, /root/reference/src/backend.rs) plus a textbook paged-decode
 * reference, used as the parity checker for the HIP backend and as the
 * `cpu_baseline` leg of bench.py.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline may load this library; the product path never does.
 *
 * Rounding contract (so results match Rust's f32 code on x86-64 Linux):
 *   - built with -ffp-contract=off and without -ffast-math: every `a*b + c`
 *     rounds twice, as Rust does (it never contracts to FMA);
 *   - sums are sequential left folds in f32, in the reference's loop order;
 *   - transcendental calls go to glibc expf/tanhf/sinf/cosf, which is what
 *     Rust's f32::exp/tanh/sin/cos lower to on this target; sqrt is the IEEE
 *     sqrtss instruction (sqrtf); powi(2)/powi(3) are x*x and (x*x)*x.
 *
 * Threading mirrors Clove's Rayon pool sized to num_cpus::get()
 * (reference src/device.rs:114-123): work is split over
 * sysconf(_SC_NPROCESSORS_ONLN) POSIX threads unless oracle_set_threads()
 * overrides it.  Per-element and per-row arithmetic does not depend on the
 * split, so results are deterministic.
 *
 * Parity pins (tests/test_oracle.py): Clove's own known-answer tests
 * (tests/engine_tests.rs:38-46, 697-706, 728-734), independent library
 * implementations in float64 (numpy matmul, torch gelu(approximate="tanh"),
 * torch softmax / layer_norm / scaled_dot_product_attention), closed forms
 * (identity and permutation matmuls, constant rows, one-hot softmax,
 * constant-V attention, ctx=1 attention) and brute-force gather indices.
 */
#define _GNU_SOURCE
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ------------------------------------------------------------------ */
/* thread pool: a fork/join split of [0, n) into contiguous chunks     */
/* ------------------------------------------------------------------ */

static int g_threads = 0;

int oracle_threads(void) {
    if (g_threads > 0) return g_threads;
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (int)n : 1;
}

void oracle_set_threads(int n) { g_threads = n; }

typedef void (*range_fn)(size_t begin, size_t end, void *ctx);

typedef struct {
    range_fn fn;
    void *ctx;
    size_t begin, end;
} job_t;

static void *job_run(void *p) {
    job_t *j = (job_t *)p;
    if (j->begin < j->end) j->fn(j->begin, j->end, j->ctx);
    return NULL;
}

static void parallel_for(size_t n, range_fn fn, void *ctx) {
    int t = oracle_threads();
    if ((size_t)t > n) t = (int)(n ? n : 1);
    if (t <= 1) {
        fn(0, n, ctx);
        return;
    }
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)t);
    job_t *jobs = (job_t *)malloc(sizeof(job_t) * (size_t)t);
    size_t chunk = (n + (size_t)t - 1) / (size_t)t;
    for (int i = 0; i < t; ++i) {
        size_t b = (size_t)i * chunk, e = b + chunk;
        if (b > n) b = n;
        if (e > n) e = n;
        jobs[i].fn = fn;
        jobs[i].ctx = ctx;
        jobs[i].begin = b;
        jobs[i].end = e;
        if (i > 0) pthread_create(&th[i], NULL, job_run, &jobs[i]);
    }
    job_run(&jobs[0]);
    for (int i = 1; i < t; ++i) pthread_join(th[i], NULL);
    free(th);
    free(jobs);
}

/* ------------------------------------------------------------------ */
/* binary elementwise ops                                              */
/* ------------------------------------------------------------------ */

typedef struct {
    const float *a, *b;
    size_t nb;
    float s;
    float *out;
    int op;
} ew_ctx;

enum { EW_ADD, EW_SUB, EW_MUL, EW_MUL_SCALAR, EW_RELU, EW_GELU, EW_SIGMOID,
       EW_TANH, EW_SIN, EW_COS };

/* sqrt(2/pi) computed in f32 exactly as backend.rs:1924 does:
 * (2.0f32 / std::f32::consts::PI).sqrt() */
static float gelu_c(void) { return sqrtf(2.0f / (float)3.14159265358979323846); }

static void ew_body(size_t begin, size_t end, void *p) {
    ew_ctx *c = (ew_ctx *)p;
    const float *a = c->a, *b = c->b;
    float *o = c->out;
    const size_t nb = c->nb;
    switch (c->op) {
    case EW_ADD: /* backend.rs:1483-1493: a[i] + b[i % b_len] */
        for (size_t i = begin; i < end; ++i) o[i] = a[i] + b[i % nb];
        break;
    case EW_SUB: /* backend.rs:1748-1758: a[i] - b[i % b_len] */
        for (size_t i = begin; i < end; ++i) o[i] = a[i] - b[i % nb];
        break;
    case EW_MUL:
        /* backend.rs:1598-1617 multiplies by b[0] when b has one element and
         * by b[i] otherwise; the WGSL branch of the same op (:1623) reads
         * b[idx % b_size].  The modulo form covers both, so it is used here. */
        for (size_t i = begin; i < end; ++i) o[i] = a[i] * b[i % nb];
        break;
    case EW_MUL_SCALAR: /* backend.rs:1686-1697 */
        for (size_t i = begin; i < end; ++i) o[i] = a[i] * c->s;
        break;
    case EW_RELU: /* backend.rs:1815-1826: if x > 0 { x } else { 0 } */
        for (size_t i = begin; i < end; ++i) o[i] = a[i] > 0.0f ? a[i] : 0.0f;
        break;
    case EW_GELU: { /* backend.rs:1917-1928 */
        const float k = gelu_c();
        for (size_t i = begin; i < end; ++i) {
            float x = a[i];
            float x3 = (x * x) * x; /* powi(3) */
            float inner = k * (x + 0.044715f * x3);
            o[i] = 0.5f * x * (1.0f + tanhf(inner));
        }
        break;
    }
    case EW_SIGMOID: /* backend.rs:2951-2960: 1 / (1 + exp(-x)) */
        for (size_t i = begin; i < end; ++i) o[i] = 1.0f / (1.0f + expf(-a[i]));
        break;
    case EW_TANH: /* backend.rs:3008-3016 */
        for (size_t i = begin; i < end; ++i) o[i] = tanhf(a[i]);
        break;
    case EW_SIN: /* backend.rs:1986-1997 */
        for (size_t i = begin; i < end; ++i) o[i] = sinf(a[i]);
        break;
    case EW_COS: /* backend.rs:2044-2055 */
        for (size_t i = begin; i < end; ++i) o[i] = cosf(a[i]);
        break;
    }
}

static void ew_run(int op, const float *a, size_t n, const float *b, size_t nb,
                   float s, float *out) {
    ew_ctx c = {a, b, nb ? nb : 1, s, out, op};
    parallel_for(n, ew_body, &c);
}

void oracle_add(const float *a, size_t n, const float *b, size_t nb, float *out) {
    ew_run(EW_ADD, a, n, b, nb, 0.f, out);
}
void oracle_sub(const float *a, size_t n, const float *b, size_t nb, float *out) {
    ew_run(EW_SUB, a, n, b, nb, 0.f, out);
}
void oracle_mul(const float *a, size_t n, const float *b, size_t nb, float *out) {
    ew_run(EW_MUL, a, n, b, nb, 0.f, out);
}
void oracle_mul_scalar(const float *a, size_t n, float s, float *out) {
    ew_run(EW_MUL_SCALAR, a, n, NULL, 1, s, out);
}
void oracle_relu(const float *a, size_t n, float *out) { ew_run(EW_RELU, a, n, NULL, 1, 0.f, out); }
void oracle_gelu(const float *a, size_t n, float *out) { ew_run(EW_GELU, a, n, NULL, 1, 0.f, out); }
void oracle_sigmoid(const float *a, size_t n, float *out) { ew_run(EW_SIGMOID, a, n, NULL, 1, 0.f, out); }
void oracle_tanh(const float *a, size_t n, float *out) { ew_run(EW_TANH, a, n, NULL, 1, 0.f, out); }
void oracle_sin(const float *a, size_t n, float *out) { ew_run(EW_SIN, a, n, NULL, 1, 0.f, out); }
void oracle_cos(const float *a, size_t n, float *out) { ew_run(EW_COS, a, n, NULL, 1, 0.f, out); }

/* ------------------------------------------------------------------ */
/* row reductions                                                      */
/* ------------------------------------------------------------------ */

typedef struct {
    const float *a, *g, *b;
    size_t cols;
    float *out;
} row_ctx;

/* backend.rs:2102-2125: max folded from -inf with f32::max, then
 * e = exp(x - max) stored and summed sequentially, then out /= sum. */
static void softmax_rows(size_t r0, size_t r1, void *p) {
    row_ctx *c = (row_ctx *)p;
    const size_t cols = c->cols;
    for (size_t i = r0; i < r1; ++i) {
        const float *x = c->a + i * cols;
        float *o = c->out + i * cols;
        float mx = -INFINITY;
        for (size_t j = 0; j < cols; ++j) mx = fmaxf(mx, x[j]); /* f32::max ignores NaN like fmaxf */
        float sum = 0.0f;
        for (size_t j = 0; j < cols; ++j) {
            float e = expf(x[j] - mx);
            o[j] = e;
            sum += e;
        }
        for (size_t j = 0; j < cols; ++j) o[j] /= sum;
    }
}

void oracle_softmax(const float *a, size_t rows, size_t cols, float *out) {
    row_ctx c = {a, NULL, NULL, cols, out};
    parallel_for(rows, softmax_rows, &c);
}

/* backend.rs:2380-2405: mean = sum/n (Iterator::sum is a sequential fold
 * starting at -0.0), var = sum((x-mean)^2)/n (biased, two-pass),
 * std = sqrt(var + 1e-5), out = ((x - mean) / std) * gamma[j] + beta[j]. */
static void layer_norm_rows(size_t r0, size_t r1, void *p) {
    row_ctx *c = (row_ctx *)p;
    const size_t cols = c->cols;
    const float n = (float)cols;
    for (size_t i = r0; i < r1; ++i) {
        const float *x = c->a + i * cols;
        float *o = c->out + i * cols;
        float s = -0.0f;
        for (size_t j = 0; j < cols; ++j) s += x[j];
        const float mean = s / n;
        float v = -0.0f;
        for (size_t j = 0; j < cols; ++j) {
            float d = x[j] - mean;
            v += d * d; /* powi(2) */
        }
        const float var = v / n;
        const float sd = sqrtf(var + 1e-5f);
        for (size_t j = 0; j < cols; ++j) o[j] = ((x[j] - mean) / sd) * c->g[j] + c->b[j];
    }
}

void oracle_layer_norm(const float *a, size_t rows, size_t cols, const float *gamma,
                       const float *beta, float *out) {
    row_ctx c = {a, gamma, beta, cols, out};
    parallel_for(rows, layer_norm_rows, &c);
}

/* ------------------------------------------------------------------ */
/* matmul                                                              */
/* ------------------------------------------------------------------ */

typedef struct {
    const float *a, *bt;
    size_t k, n;
    float *c;
} mm_ctx;

static void mm_rows(size_t r0, size_t r1, void *p) {
    mm_ctx *c = (mm_ctx *)p;
    for (size_t i = r0; i < r1; ++i) {
        const float *ra = c->a + i * c->k;
        float *row = c->c + i * c->n;
        for (size_t j = 0; j < c->n; ++j) {
            const float *rb = c->bt + j * c->k;
            float sum = 0.0f;
            for (size_t q = 0; q < c->k; ++q) sum += ra[q] * rb[q];
            row[j] = sum;
        }
    }
}

/* backend.rs:266-287 (rayon_matmul): B is transposed first, then each output
 * row is computed in parallel; each element is a sequential f32 dot product
 * over p = 0..k with separate multiply and add roundings.  `row_begin` and
 * `row_end` restrict the rows computed (the bench times a bounded sample);
 * pass 0 and m for the whole product. */
void oracle_matmul_rows(const float *a, const float *b, size_t m, size_t k, size_t n,
                        size_t row_begin, size_t row_end, float *c) {
    (void)m;
    float *bt = (float *)malloc(sizeof(float) * k * n);
    for (size_t i = 0; i < k; ++i)
        for (size_t j = 0; j < n; ++j) bt[j * k + i] = b[i * n + j];
    mm_ctx ctx = {a + row_begin * k, bt, k, n, c + row_begin * n};
    parallel_for(row_end - row_begin, mm_rows, &ctx);
    free(bt);
}

void oracle_matmul(const float *a, const float *b, size_t m, size_t k, size_t n, float *c) {
    oracle_matmul_rows(a, b, m, k, n, 0, m, c);
}

/* ------------------------------------------------------------------ */
/* paged decode attention                                              */
/* ------------------------------------------------------------------ */
/*
 * Clove has no CPU paged attention (backend.rs:2937-2948 panics, the WGSL at
 * lazy.rs:5241-5275 is a placeholder), so this is the textbook definition on
 * the layout Clove documents for its cache (nn.rs:534-535):
 *   kv_cache  : two planes [2][num_blocks][block_size][H][D] (plane 0 = K,
 *               plane 1 = V), f32
 *   block_tables : int32 [B][max_blocks]
 *   context_lens : int32 [B]
 *   q, k_new, v_new, out : [B][H*D]
 * For sequence b the context is tokens t = 0..ctx_b-1.  Token t lives in
 * physical slot bt[b][t / block_size] * block_size + t % block_size.  When
 * k_new/v_new are given, the last token (t = ctx_b-1) is taken from them
 * instead of from the cache (the freshly projected token of nn.rs:540-546).
 * out = sum_t softmax_t(scale * q.k_t) v_t; ctx_b == 0 gives zeros.
 * The f32 variant follows Clove's softmax order (backend.rs:2107-2124):
 * sequential dot, max fold, exp, sequential sum, divide, then a sequential
 * weighted sum over t.
 */

typedef struct {
    const float *q, *kn, *vn, *kv;
    const int32_t *bt, *cl;
    int64_t num_blocks;
    int H, D, bs, max_blocks;
    float scale;
    float *out;
    double *out64;
} pa_ctx;

static inline const float *pa_row(const pa_ctx *c, int plane, int b, int t, int h, int ctx) {
    if (c->kn && t == ctx - 1) {
        const float *src = plane ? c->vn : c->kn;
        return src + ((size_t)b * c->H + h) * c->D;
    }
    int64_t blk = c->bt[(size_t)b * c->max_blocks + t / c->bs];
    int64_t slot = blk * c->bs + t % c->bs;
    size_t plane_off = (size_t)plane * (size_t)c->num_blocks * c->bs * c->H * c->D;
    return c->kv + plane_off + ((size_t)slot * c->H + h) * c->D;
}

static void pa_body_f32(size_t p0, size_t p1, void *p) {
    pa_ctx *c = (pa_ctx *)p;
    float *s = NULL;
    size_t s_cap = 0;
    for (size_t pair = p0; pair < p1; ++pair) {
        int b = (int)(pair / c->H), h = (int)(pair % c->H);
        int ctx = c->cl[b];
        const float *q = c->q + ((size_t)b * c->H + h) * c->D;
        float *o = c->out + ((size_t)b * c->H + h) * c->D;
        for (int d = 0; d < c->D; ++d) o[d] = 0.0f;
        if (ctx <= 0) continue;
        if ((size_t)ctx > s_cap) {
            free(s);
            s_cap = (size_t)ctx;
            s = (float *)malloc(sizeof(float) * s_cap);
        }
        float mx = -INFINITY;
        for (int t = 0; t < ctx; ++t) {
            const float *k = pa_row(c, 0, b, t, h, ctx);
            float dot = 0.0f;
            for (int d = 0; d < c->D; ++d) dot += q[d] * k[d];
            s[t] = dot * c->scale;
            mx = fmaxf(mx, s[t]);
        }
        float sum = 0.0f;
        for (int t = 0; t < ctx; ++t) {
            s[t] = expf(s[t] - mx);
            sum += s[t];
        }
        for (int t = 0; t < ctx; ++t) s[t] /= sum;
        for (int t = 0; t < ctx; ++t) {
            const float *v = pa_row(c, 1, b, t, h, ctx);
            for (int d = 0; d < c->D; ++d) o[d] += s[t] * v[d];
        }
    }
    free(s);
}

static void pa_body_f64(size_t p0, size_t p1, void *p) {
    pa_ctx *c = (pa_ctx *)p;
    double *s = NULL;
    size_t s_cap = 0;
    for (size_t pair = p0; pair < p1; ++pair) {
        int b = (int)(pair / c->H), h = (int)(pair % c->H);
        int ctx = c->cl[b];
        const float *q = c->q + ((size_t)b * c->H + h) * c->D;
        double *o = c->out64 + ((size_t)b * c->H + h) * c->D;
        for (int d = 0; d < c->D; ++d) o[d] = 0.0;
        if (ctx <= 0) continue;
        if ((size_t)ctx > s_cap) {
            free(s);
            s_cap = (size_t)ctx;
            s = (double *)malloc(sizeof(double) * s_cap);
        }
        double mx = -INFINITY;
        for (int t = 0; t < ctx; ++t) {
            const float *k = pa_row(c, 0, b, t, h, ctx);
            double dot = 0.0;
            for (int d = 0; d < c->D; ++d) dot += (double)q[d] * (double)k[d];
            s[t] = dot * (double)c->scale;
            if (s[t] > mx) mx = s[t];
        }
        double sum = 0.0;
        for (int t = 0; t < ctx; ++t) {
            s[t] = exp(s[t] - mx);
            sum += s[t];
        }
        for (int t = 0; t < ctx; ++t) {
            const float *v = pa_row(c, 1, b, t, h, ctx);
            const double w = s[t] / sum;
            for (int d = 0; d < c->D; ++d) o[d] += w * (double)v[d];
        }
    }
    free(s);
}

/* Sequences [seq_begin, seq_end) are computed; rows of other sequences in
 * `out` are left untouched (the bench times a bounded sample). */
void oracle_paged_attention_f32(const float *q, const float *k_new, const float *v_new,
                                const float *kv_cache, int64_t num_blocks,
                                const int32_t *block_tables, int max_blocks,
                                const int32_t *context_lens, int num_seqs, int num_heads,
                                int head_dim, int block_size, float scale, int seq_begin,
                                int seq_end, float *out) {
    (void)num_seqs;
    pa_ctx c = {q, k_new, v_new, kv_cache, block_tables, context_lens, num_blocks,
                num_heads, head_dim, block_size, max_blocks, scale, out, NULL};
    /* shift the base pointers so that pair index 0 is (seq_begin, head 0) */
    size_t row = (size_t)seq_begin * num_heads * head_dim;
    c.q = q + row;
    c.kn = k_new ? k_new + row : NULL;
    c.vn = v_new ? v_new + row : NULL;
    c.bt = block_tables + (size_t)seq_begin * max_blocks;
    c.cl = context_lens + seq_begin;
    c.out = out + row;
    parallel_for((size_t)(seq_end - seq_begin) * num_heads, pa_body_f32, &c);
}

void oracle_paged_attention_f64(const float *q, const float *k_new, const float *v_new,
                                const float *kv_cache, int64_t num_blocks,
                                const int32_t *block_tables, int max_blocks,
                                const int32_t *context_lens, int num_seqs, int num_heads,
                                int head_dim, int block_size, float scale, double *out) {
    pa_ctx c = {q, k_new, v_new, kv_cache, block_tables, context_lens, num_blocks,
                num_heads, head_dim, block_size, max_blocks, scale, NULL, out};
    parallel_for((size_t)num_seqs * num_heads, pa_body_f64, &c);
}

/* Physical token slot of every logical token: slots[b][t] =
 * bt[b][t / bs] * bs + t % bs for t < ctx_b, -1 beyond (the gather the
 * reference WGSL performs at lazy.rs:5262-5270, with the table stride taken
 * from the table's shape instead of the hard-coded 1024). */
void oracle_paged_slots(const int32_t *block_tables, int max_blocks, const int32_t *context_lens,
                        int num_seqs, int block_size, int max_ctx, int32_t *slots) {
    for (int b = 0; b < num_seqs; ++b)
        for (int t = 0; t < max_ctx; ++t)
            slots[(size_t)b * max_ctx + t] =
                t < context_lens[b]
                    ? block_tables[(size_t)b * max_blocks + t / block_size] * block_size + t % block_size
                    : -1;
}

/* ------------------------------------------------------------------ */
/* backward passes and losses (the autograd closures of backend.rs)    */
/* ------------------------------------------------------------------ */

typedef struct {
    const float *x, *g;
    float *out;
    float s;
} bw_ctx;

/* backend.rs:1858-1870 (relu backward): p_grad[i] = out[i] > 0 ? g[i] : 0
 * with out = relu(x); out > 0 exactly when x > 0, so x may be passed. */
static void relu_bw_body(size_t b, size_t e, void *p) {
    bw_ctx *c = (bw_ctx *)p;
    for (size_t i = b; i < e; ++i) c->out[i] = c->x[i] > 0.0f ? c->g[i] : 0.0f;
}
void oracle_relu_backward(const float *x, const float *g, size_t n, float *out) {
    bw_ctx c = {x, g, out, 0.f};
    parallel_for(n, relu_bw_body, &c);
}

/* backend.rs:1965-1981 (gelu backward), left to right as Rust evaluates it:
 *   c = (2/pi).sqrt(); inner = c * (x + 0.044715 * x.powi(3));
 *   sech2 = 1 - inner.tanh().powi(2);
 *   d = 0.5 * (1 + inner.tanh()) + 0.5 * x * sech2 * c * (1 + 3.0 * 0.044715 * x.powi(2));
 *   p_grad = g * d
 * 3.0 * 0.044715 is folded in f32 before it meets x*x, as Rust folds it. */
static void gelu_bw_body(size_t b, size_t e, void *p) {
    bw_ctx *c = (bw_ctx *)p;
    const float k = gelu_c();
    const float k3 = 3.0f * 0.044715f;
    for (size_t i = b; i < e; ++i) {
        const float x = c->x[i];
        const float x3 = (x * x) * x;
        const float t = tanhf(k * (x + 0.044715f * x3));
        const float sech2 = 1.0f - t * t;
        const float d = 0.5f * (1.0f + t) + 0.5f * x * sech2 * k * (1.0f + k3 * (x * x));
        c->out[i] = c->g[i] * d;
    }
}
void oracle_gelu_backward(const float *x, const float *g, size_t n, float *out) {
    bw_ctx c = {x, g, out, 0.f};
    parallel_for(n, gelu_bw_body, &c);
}

/* backend.rs:2163-2183 (softmax backward): s = sum_j dy[j]*y[j] as a
 * sequential fold, then dx[j] = y[j] * (dy[j] - s). */
static void softmax_bw_rows(size_t r0, size_t r1, void *p) {
    row_ctx *c = (row_ctx *)p;
    const size_t cols = c->cols;
    for (size_t i = r0; i < r1; ++i) {
        const float *y = c->a + i * cols, *dy = c->g + i * cols;
        float *o = c->out + i * cols;
        float s = 0.0f;
        for (size_t j = 0; j < cols; ++j) s += dy[j] * y[j];
        for (size_t j = 0; j < cols; ++j) o[j] = y[j] * (dy[j] - s);
    }
}
void oracle_softmax_backward(const float *y, const float *dy, size_t rows, size_t cols,
                             float *dx) {
    row_ctx c = {y, dy, NULL, cols, dx};
    parallel_for(rows, softmax_bw_rows, &c);
}

/* backend.rs:1314-1360 (matmul backward), both loops sequential f32 dots:
 *   dA[r][c] = sum_{i<n} dC[r*n + i] * B[c*n + i]     (dA = dC . B^T, m x k)
 *   dB[r][c] = sum_{i<m} A[i*k + r] * dC[i*n + c]     (dB = A^T . dC, k x n)
 * Rows [r0, r1) of each are computed (a bounded sample for the baseline). */
typedef struct {
    const float *a, *b, *dc;
    size_t m, k, n;
    float *out;
} mmb_ctx;
static void mmb_da_rows(size_t r0, size_t r1, void *p) {
    mmb_ctx *c = (mmb_ctx *)p;
    for (size_t r = r0; r < r1; ++r)
        for (size_t col = 0; col < c->k; ++col) {
            float s = 0.0f;
            for (size_t i = 0; i < c->n; ++i) s += c->dc[r * c->n + i] * c->b[col * c->n + i];
            c->out[r * c->k + col] = s;
        }
}
static void mmb_db_rows(size_t r0, size_t r1, void *p) {
    mmb_ctx *c = (mmb_ctx *)p;
    for (size_t r = r0; r < r1; ++r)
        for (size_t col = 0; col < c->n; ++col) {
            float s = 0.0f;
            for (size_t i = 0; i < c->m; ++i) s += c->a[i * c->k + r] * c->dc[i * c->n + col];
            c->out[r * c->n + col] = s;
        }
}
typedef struct {
    range_fn fn;
    mmb_ctx *c;
    size_t r0;
} offset_ctx;
static void offset_body(size_t b, size_t e, void *p) {
    offset_ctx *o = (offset_ctx *)p;
    o->fn(o->r0 + b, o->r0 + e, o->c);
}
void oracle_matmul_backward_rows(const float *a, const float *b, const float *dc, size_t m,
                                 size_t k, size_t n, size_t da_r0, size_t da_r1, size_t db_r0,
                                 size_t db_r1, float *da, float *db) {
    mmb_ctx c1 = {a, b, dc, m, k, n, da};
    offset_ctx o1 = {mmb_da_rows, &c1, da_r0};
    if (da && da_r1 > da_r0) parallel_for(da_r1 - da_r0, offset_body, &o1);
    mmb_ctx c2 = {a, b, dc, m, k, n, db};
    offset_ctx o2 = {mmb_db_rows, &c2, db_r0};
    if (db && db_r1 > db_r0) parallel_for(db_r1 - db_r0, offset_body, &o2);
}

/* backend.rs:1527-1538 (add backward, b operand): gb[i % nb] += g[i] over
 * i in order; backend.rs:1800-1810 (sub): gb[i % nb] -= g[i].  One thread:
 * the fold order is the reference's. */
void oracle_bias_grad(const float *g, size_t n, size_t nb, int negate, float *gb) {
    for (size_t j = 0; j < nb; ++j) gb[j] = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        if (negate) gb[i % nb] -= g[i];
        else gb[i % nb] += g[i];
    }
}

/* Rust's `f32 as usize` saturates: NaN and negatives give 0. */
static size_t target_index(float v) {
    if (!(v > 0.0f)) return 0;
    if (v >= 18446744073709551615.0f) return (size_t)-1;
    return (size_t)v;
}

/* backend.rs:2661-2680 (cross entropy): per row, max folded from -inf,
 * sum_exp = sum exp(l - max) sequentially, total -= (l[t] - max) - ln(sum_exp)
 * over rows in order; loss = total / rows.  Only the first
 * min(rows, ntargets) rows contribute (`targets.iter().enumerate().take(rows)`).
 * Returns -1 (Rust would panic indexing the row) when a target is >= cols. */
int oracle_cross_entropy(const float *logits, const float *targets, size_t ntargets,
                         size_t rows, size_t cols, float *loss) {
    float total = 0.0f;
    const size_t used = ntargets < rows ? ntargets : rows;
    for (size_t i = 0; i < used; ++i) {
        const float *l = logits + i * cols;
        float mx = -INFINITY;
        for (size_t j = 0; j < cols; ++j) mx = fmaxf(mx, l[j]);
        float s = 0.0f;
        for (size_t j = 0; j < cols; ++j) s += expf(l[j] - mx);
        const size_t t = target_index(targets[i]);
        if (t >= cols) return -1;
        total -= (l[t] - mx) - logf(s);
    }
    *loss = total / (float)rows;
    return 0;
}

/* backend.rs:2686-2712 (cross entropy backward): per row, the same max and
 * exps (stored, summed sequentially), prob = exps[j] / sum_exp and
 * grad = (prob - [j == t]) * g / rows, evaluated left to right; rows past
 * the targets keep a zero gradient. */
int oracle_cross_entropy_backward(const float *logits, const float *targets, size_t ntargets,
                                  size_t rows, size_t cols, float g, float *grad) {
    const size_t used = ntargets < rows ? ntargets : rows;
    memset(grad, 0, rows * cols * sizeof(float));
    for (size_t i = 0; i < used; ++i) {
        const float *l = logits + i * cols;
        float *o = grad + i * cols;
        float mx = -INFINITY;
        for (size_t j = 0; j < cols; ++j) mx = fmaxf(mx, l[j]);
        float s = 0.0f;
        for (size_t j = 0; j < cols; ++j) {
            o[j] = expf(l[j] - mx);
            s += o[j];
        }
        const size_t t = target_index(targets[i]);
        if (t >= cols) return -1;
        for (size_t j = 0; j < cols; ++j) {
            const float prob = o[j] / s;
            const float tv = j == t ? 1.0f : 0.0f;
            o[j] = (prob - tv) * g / (float)rows;
        }
    }
    return 0;
}

/* backend.rs:2765-2772 (mse): sum of (p - t).powi(2) as a sequential fold,
 * divided by n. */
float oracle_mse(const float *p, const float *t, size_t n) {
    float s = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        const float d = p[i] - t[i];
        s += d * d;
    }
    return s / (float)n;
}

/* backend.rs:2780-2790 (mse backward): grad = 2.0 * (p - t) * g / n. */
void oracle_mse_backward(const float *p, const float *t, size_t n, float g, float *grad) {
    const float nf = (float)n;
    for (size_t i = 0; i < n; ++i) grad[i] = 2.0f * (p[i] - t[i]) * g / nf;
}

/* ------------------------------------------------------------------ */
/* AdamW (optim.rs:375-395, the Rayon branch of AdamW::step)          */
/* ------------------------------------------------------------------ */

typedef struct {
    float *w, *m, *v;
    const float *g;
    float lr, b1, b2, eps, wd, scale, clip, bc1, bc2;
} adamw_ctx;

/* Rust's f32::clamp: NaN passes through. */
static float clamp_rs(float x, float lo, float hi) {
    if (x < lo) x = lo;
    if (x > hi) x = hi;
    return x;
}

/* Per element, in Rust's evaluation order:
 *   w -= lr * wd * w;  g' = clamp(g / scale, -clip, clip);
 *   m = b1 * m + (1 - b1) * g';  v = b2 * v + (1 - b2) * g' * g';
 *   w -= lr * (m / (1 - b1^t)) / (sqrt(v / (1 - b2^t)) + eps)
 * with 1 - b^t (powf) computed once by the caller, as t is per step. */
static void adamw_body(size_t b, size_t e, void *p) {
    adamw_ctx *c = (adamw_ctx *)p;
    for (size_t i = b; i < e; ++i) {
        float w = c->w[i];
        w -= c->lr * c->wd * w;
        const float gu = c->g[i] / c->scale;
        const float g = clamp_rs(gu, -c->clip, c->clip);
        const float m = c->b1 * c->m[i] + (1.0f - c->b1) * g;
        const float v = c->b2 * c->v[i] + (1.0f - c->b2) * g * g;
        c->m[i] = m;
        c->v[i] = v;
        const float m_hat = m / c->bc1;
        const float v_hat = v / c->bc2;
        w -= c->lr * m_hat / (sqrtf(v_hat) + c->eps);
        c->w[i] = w;
    }
}

/* In place on w, m, v.  step is AdamW::step_count after its increment. */
void oracle_adamw(float *w, const float *g, float *m, float *v, size_t n, float lr, float b1,
                  float b2, float eps, float wd, float scale, float clip, uint32_t step) {
    const float t = (float)step;
    adamw_ctx c = {w, m, v, g, lr, b1, b2, eps, wd, scale, clip,
                   1.0f - powf(b1, t), 1.0f - powf(b2, t)};
    parallel_for(n, adamw_body, &c);
}

/* ------------------------------------------------------------------ */
/* RoPE and attention prefill                                          */
/* ------------------------------------------------------------------ */

/* backend.rs:2797-2826 (rope): x is [batch, seq, hidden], heads of head_dim
 * (even) dims, hidden / head_dim whole heads; pair (i, i+1) of each head at
 * position pos rotates by
 * theta = (pos + pos_offset) / 10000^(i / head_dim), all in f32:
 *   x1' = x1 cos - x2 sin,  x2' = x1 sin + x2 cos. */
typedef struct {
    const float *x;
    float *out;
    size_t seq, hidden, head_dim, pos_offset;
} rope_ctx;
static void rope_rows(size_t r0, size_t r1, void *p) {
    rope_ctx *c = (rope_ctx *)p;
    for (size_t r = r0; r < r1; ++r) {  /* r = b * seq + pos */
        const size_t pos = r % c->seq;
        const float ap = (float)(pos + c->pos_offset);
        const float *x = c->x + r * c->hidden;
        float *o = c->out + r * c->hidden;
        for (size_t h = 0; h + c->head_dim <= c->hidden; h += c->head_dim)
            for (size_t i = 0; i < c->head_dim; i += 2) {
                const float theta = ap / powf(10000.0f, (float)i / (float)c->head_dim);
                const float x1 = x[h + i], x2 = x[h + i + 1];
                o[h + i] = x1 * cosf(theta) - x2 * sinf(theta);
                o[h + i + 1] = x1 * sinf(theta) + x2 * cosf(theta);
            }
    }
}
void oracle_rope(const float *x, size_t batch, size_t seq, size_t hidden, size_t head_dim,
                 size_t pos_offset, float *out) {
    /* result starts as zeros (backend.rs:2800): dims past the last whole head stay 0 */
    memset(out, 0, batch * seq * hidden * sizeof(float));
    rope_ctx c = {x, out, seq, hidden, head_dim, pos_offset};
    parallel_for(batch * seq, rope_rows, &c);
}

/* Attention prefill, the computation lazy.rs:4821-4909 fuses (FlashAttention
 * step, pattern lazy.rs:1621-1690) with an exact exp: q [B, S, H*D], k and v
 * [B, Sk, H*D]; with ATTN_ROPE q and k are rotated first (positions s + q_pos
 * and t + k_pos); score_t = (q . k_t, a sequential f32 dot) * scale, keys
 * with t + k_pos > s + q_pos skipped under ATTN_CAUSAL; the softmax is
 * backend.rs:2102-2125's (max fold, exp, sequential sum, divide) and
 * out = sum_t p_t v_t summed in key order.  A row with no key gets 0. */
enum { ATTN_CAUSAL = 1, ATTN_ROPE = 2 };
typedef struct {
    const float *q, *k, *v;
    float *out;
    size_t S, Sk, H, D, s_lo, s_hi;
    long q_pos, k_pos;
    int flags;
    float scale;
} attn_ctx;
static void attn_rows(size_t r0, size_t r1, void *p) {
    attn_ctx *c = (attn_ctx *)p;
    const size_t H = c->H, D = c->D, HD = H * D, ns = c->s_hi - c->s_lo;
    float *sc = (float *)malloc(c->Sk * sizeof(float));
    for (size_t r = r0; r < r1; ++r) { /* r = (b * H + h) * ns + (s - s_lo) */
        const size_t s = c->s_lo + r % ns, bh = r / ns, h = bh % H, b = bh / H;
        const float *q = c->q + (b * c->S + s) * HD + h * D;
        const float *kb = c->k + b * c->Sk * HD + h * D;
        const float *vb = c->v + b * c->Sk * HD + h * D;
        float *o = c->out + (b * c->S + s) * HD + h * D;
        float mx = -INFINITY;
        size_t nk = 0;
        for (size_t t = 0; t < c->Sk; ++t) {
            if ((c->flags & ATTN_CAUSAL) && (long)t + c->k_pos > (long)s + c->q_pos) {
                sc[t] = -INFINITY;
                continue;
            }
            float dot = 0.0f;
            const float *kt = kb + t * HD;
            for (size_t d = 0; d < D; ++d) dot += q[d] * kt[d];
            sc[t] = dot * c->scale;
            mx = fmaxf(mx, sc[t]);
            ++nk;
        }
        if (nk == 0) {
            for (size_t d = 0; d < D; ++d) o[d] = 0.0f;
            continue;
        }
        float sum = 0.0f;
        for (size_t t = 0; t < c->Sk; ++t) {
            const float e = sc[t] == -INFINITY ? 0.0f : expf(sc[t] - mx);
            sc[t] = e;
            sum += e;
        }
        for (size_t t = 0; t < c->Sk; ++t) sc[t] /= sum;
        for (size_t d = 0; d < D; ++d) {
            float acc = 0.0f;
            for (size_t t = 0; t < c->Sk; ++t)
                if (sc[t] != 0.0f) acc += sc[t] * vb[t * HD + d];
            o[d] = acc;
        }
    }
    free(sc);
}

/* q and k rotated once (the same per-element f32 operations as rope above,
 * at positions s + q_pos / t + k_pos), then plain attention for the query
 * rows [s_lo, s_hi) of every (batch, head); other rows of out are left. */
void oracle_attention(const float *q, const float *k, const float *v, size_t B, size_t S,
                      size_t Sk, size_t H, size_t D, long q_pos, long k_pos, int flags,
                      float scale, size_t s_lo, size_t s_hi, float *out) {
    const size_t HD = H * D;
    float *qr = NULL, *kr = NULL;
    if (flags & ATTN_ROPE) {
        qr = (float *)malloc(B * S * HD * sizeof(float));
        kr = (float *)malloc(B * Sk * HD * sizeof(float));
        /* HD is a whole number of heads, so every element is rotated */
        rope_ctx cq = {q, qr, S, HD, D, (size_t)q_pos};
        parallel_for(B * S, rope_rows, &cq);
        rope_ctx ck = {k, kr, Sk, HD, D, (size_t)k_pos};
        parallel_for(B * Sk, rope_rows, &ck);
        q = qr;
        k = kr;
    }
    if (s_hi > S) s_hi = S;
    if (s_lo < s_hi) {
        attn_ctx c = {q, k, v, out, S, Sk, H, D, s_lo, s_hi, q_pos, k_pos, flags, scale};
        parallel_for(B * H * (s_hi - s_lo), attn_rows, &c);
    }
    free(qr);
    free(kr);
}
