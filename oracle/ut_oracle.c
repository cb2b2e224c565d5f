/*
 * ut_oracle.c -- CPU restatement of the undertow reference's MTP decode path.
 *
 * TEST INFRASTRUCTURE ONLY (see ut_oracle.h).  Never linked into the product
 * library; the HIP path must fail loudly rather than fall back to this code.
 *
 * Build: gcc -O2 -ffp-contract=off -fPIC -shared (oracle/Makefile).  The
 * -ffp-contract=off flag matters: the Rust reference never fuses a*b+c, so a
 * contracted build would not be the same arithmetic.
 */
#define _DEFAULT_SOURCE /* madvise */
#include "ut_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>

#if defined(__FP_FAST_FMAF) && !defined(UTO_ALLOW_FMA)
/* An FMA-contracting build would not restate the reference's arithmetic. */
#endif

static void *xcalloc(size_t n, size_t sz) {
    void *p = calloc(n ? n : 1, sz ? sz : 1);
    if (!p) { fprintf(stderr, "ut_oracle: out of memory\n"); abort(); }
    return p;
}

/* ===================================================================== RNG */
/* Pcg32::new / next_u32 / uniform / normal (undertow-bench/src/rng.rs:15-47). */
uint32_t uto_pcg32_next(uto_pcg32 *r) {
    uint64_t old = r->state;
    r->state = old * 6364136223846793005ULL + r->inc;
    uint32_t xorshifted = (uint32_t)(((old >> 18) ^ old) >> 27);
    uint32_t rot = (uint32_t)(old >> 59);
    return (xorshifted >> rot) | (xorshifted << ((32u - rot) & 31u));
}

void uto_pcg32_init(uto_pcg32 *r, uint64_t seed, uint64_t stream) {
    r->state = 0;
    r->inc = (stream << 1) | 1u;
    (void)uto_pcg32_next(r);
    r->state += seed;
    (void)uto_pcg32_next(r);
}

float uto_pcg32_uniform(uto_pcg32 *r) {
    return (float)(uto_pcg32_next(r) >> 8) * (1.0f / 16777216.0f);
}

float uto_pcg32_normal(uto_pcg32 *r) {
    float acc = 0.0f;
    for (int i = 0; i < 12; i++) acc += uto_pcg32_uniform(r);
    return acc - 6.0f;
}

void uto_pcg32_fill(uint64_t seed, uint64_t stream, int kind, float std,
                    float *out, int64_t n) {
    uto_pcg32 r;
    uto_pcg32_init(&r, seed, stream);
    for (int64_t i = 0; i < n; i++)
        out[i] = kind == 0 ? uto_pcg32_uniform(&r) : uto_pcg32_normal(&r) * std;
}

/* =================================================================== quant */
int8_t uto_unpack_i4(const uint8_t *row, int64_t i) {
    /* kernels.rs:10-19: low nibble holds the even index; 4-bit two's
     * complement sign extension. */
    uint8_t b = row[i / 2];
    uint8_t nib = (i % 2 == 0) ? (uint8_t)(b & 0x0F) : (uint8_t)(b >> 4);
    return (int8_t)((int8_t)(nib << 4) >> 4);
}

int64_t uto_payload_bytes(int fmt, int64_t out_dim, int64_t in_dim) {
    switch (fmt) {
    case UTO_F32: return out_dim * in_dim * 4;
    case UTO_INT8: return out_dim * in_dim;
    default: return out_dim * ((in_dim + 1) / 2);
    }
}

static float row_absmax(const float *row, int64_t n) {
    /* fold(0, |m, v| m.max(v.abs())) */
    float m = 0.0f;
    for (int64_t i = 0; i < n; i++) m = fmaxf(m, fabsf(row[i]));
    return m;
}

int uto_quantize(int fmt, const float *w, int64_t out_dim, int64_t in_dim,
                 void *payload, float *scales) {
    /* qtensor.rs:142-213 */
    for (int64_t k = 0; k < out_dim * in_dim; k++)
        if (!isfinite(w[k])) return -1;
    if (fmt == UTO_F32) {
        memcpy(payload, w, (size_t)(out_dim * in_dim) * 4);
        return 0;
    }
    if (fmt == UTO_INT8) {
        int8_t *q = (int8_t *)payload;
        memset(q, 0, (size_t)(out_dim * in_dim));
        for (int64_t o = 0; o < out_dim; o++) {
            const float *row = w + o * in_dim;
            float max = row_absmax(row, in_dim);
            scales[o] = 0.0f;
            if (max > 0.0f) {
                float s = max / 127.0f;
                scales[o] = s;
                for (int64_t i = 0; i < in_dim; i++) {
                    float v = roundf(row[i] / s);
                    v = v < -127.0f ? -127.0f : (v > 127.0f ? 127.0f : v);
                    q[o * in_dim + i] = (int8_t)v;
                }
            }
        }
        return 0;
    }
    int64_t rb = (in_dim + 1) / 2;
    uint8_t *packed = (uint8_t *)payload;
    memset(packed, 0, (size_t)(out_dim * rb));
    for (int64_t o = 0; o < out_dim; o++) {
        const float *row = w + o * in_dim;
        float max = row_absmax(row, in_dim);
        scales[o] = 0.0f;
        if (max > 0.0f) {
            float s = max / 7.0f;
            scales[o] = s;
            for (int64_t i = 0; i < in_dim; i++) {
                float v = roundf(row[i] / s);
                v = v < -7.0f ? -7.0f : (v > 7.0f ? 7.0f : v);
                uint8_t nib = (uint8_t)((int8_t)v) & 0x0F;
                uint8_t *byte = &packed[o * rb + i / 2];
                if (i % 2 == 0) *byte |= nib;
                else *byte |= (uint8_t)(nib << 4);
            }
        }
    }
    return 0;
}

/* lib.rs:46-59 */
float uto_quantize_activations(const float *x, int64_t n, int8_t *out) {
    float max = 0.0f;
    for (int64_t i = 0; i < n; i++) {
        /* f32::max returns the other operand when one is NaN */
        const float a = fabsf(x[i]);
        if (!(a <= max) && !isnan(a)) max = a;
    }
    if (max == 0.0f) {
        memset(out, 0, (size_t)n);
        return 0.0f;
    }
    const float scale = max / 127.0f;
    const float inv = 127.0f / max;
    for (int64_t i = 0; i < n; i++) {
        float t = roundf(x[i] * inv);
        /* clamp keeps NaN; `as i8` maps NaN to 0 */
        if (isnan(t)) {
            out[i] = 0;
            continue;
        }
        t = t < -127.0f ? -127.0f : t > 127.0f ? 127.0f : t;
        out[i] = (int8_t)t;
    }
    return scale;
}

/* avx512.rs:221-242: per row, the activations quantised once, then for
 * every output row the exact integer dot (dot_i8_vnni's total - 128 * sum_b
 * + tail is the plain sum of products) as f32 times a_scale times scale. */
void uto_matmul_fast_i8(const int8_t *q, const float *scales, int64_t out_dim, int64_t in_dim,
                        const float *x, int64_t seq, float *out) {
    int8_t *qa = (int8_t *)malloc((size_t)(in_dim > 0 ? in_dim : 1));
    for (int64_t s = 0; s < seq; s++) {
        const float a_scale = uto_quantize_activations(x + s * in_dim, in_dim, qa);
        for (int64_t o = 0; o < out_dim; o++) {
            const int8_t *row = q + o * in_dim;
            int32_t acc = 0;
            for (int64_t i = 0; i < in_dim; i++) acc += (int32_t)qa[i] * (int32_t)row[i];
            out[s * out_dim + o] = ((float)acc * a_scale) * scales[o];
        }
    }
    free(qa);
}

void uto_add_scaled_row(int fmt, const void *payload, const float *scales,
                        int64_t out_dim, int64_t in_dim, int64_t row,
                        float factor, float *acc) {
    (void)out_dim;
    if (fmt == UTO_F32) {
        const float *r = (const float *)payload + row * in_dim;
        for (int64_t i = 0; i < in_dim; i++) acc[i] += factor * r[i];
    } else if (fmt == UTO_INT8) {
        float s = factor * scales[row];
        const int8_t *r = (const int8_t *)payload + row * in_dim;
        for (int64_t i = 0; i < in_dim; i++) acc[i] += s * (float)r[i];
    } else {
        float s = factor * scales[row];
        const uint8_t *r = (const uint8_t *)payload + row * ((in_dim + 1) / 2);
        for (int64_t i = 0; i < in_dim; i++) acc[i] += s * (float)uto_unpack_i4(r, i);
    }
}

void uto_dequantize(int fmt, const void *payload, const float *scales,
                    int64_t out_dim, int64_t in_dim, float *out) {
    memset(out, 0, (size_t)(out_dim * in_dim) * 4);
    for (int64_t r = 0; r < out_dim; r++)
        uto_add_scaled_row(fmt, payload, scales, out_dim, in_dim, r, 1.0f,
                           out + r * in_dim);
}

#ifdef UTO_SIMD_MATMUL
/* The CPU baseline build (oracle/Makefile: libcpu_model.so): integer
 * matmuls go to the restated dispatched kernels with the rayon row split
 * (cpu_baseline.c: avx512.rs / avx2.rs, qtensor.rs:281-319), as the
 * reference's QTensor::matmul dispatches them at run time.  The parity
 * checker (liboracle.so) never defines this. */
void ucb_matmul(int fmt, const void *payload, const float *scales, int64_t out_dim, int64_t in_dim,
                const float *x, int64_t seq, float *out, int nthreads);
#endif

/* FAST_INT8 (undertow-quant/src/lib.rs:31-43): process-global, off by
 * default; QTensor::matmul on Int8 takes the fast path while it is set
 * (qtensor.rs:385-398). */
static int g_fast_int8 = 0;
void uto_set_fast_int8(int on) { g_fast_int8 = on != 0; }
int uto_fast_int8_enabled(void) { return g_fast_int8; }

void uto_matmul(int fmt, const void *payload, const float *scales,
                int64_t out_dim, int64_t in_dim, const float *x, int64_t seq,
                float *out) {
    if (g_fast_int8 && fmt == UTO_INT8) {
        uto_matmul_fast_i8((const int8_t *)payload, scales, out_dim, in_dim, x, seq, out);
        return;
    }
#ifdef UTO_SIMD_MATMUL
    if (fmt != UTO_F32) {
        ucb_matmul(fmt, payload, scales, out_dim, in_dim, x, seq, out, 0);
        return;
    }
#endif
    /* Rows are independent and each keeps its sequential order, so the
     * thread split changes no value (the reference's rayon row split,
     * qtensor.rs:274-309). */
    for (int64_t s = 0; s < seq; s++) {
        const float *xs = x + s * in_dim;
        float *os = out + s * out_dim;
#pragma omp parallel for schedule(static) if (out_dim * in_dim >= (1 << 18))
        for (int64_t o = 0; o < out_dim; o++) {
            float acc = 0.0f;
            if (fmt == UTO_F32) {
                /* lib.rs:128-144: no scale */
                const float *wr = (const float *)payload + o * in_dim;
                for (int64_t i = 0; i < in_dim; i++) acc += xs[i] * wr[i];
                os[o] = acc;
            } else if (fmt == UTO_INT8) {
                /* kernels.rs:21-44 */
                const int8_t *row = (const int8_t *)payload + o * in_dim;
                for (int64_t i = 0; i < in_dim; i++) acc += xs[i] * (float)row[i];
                os[o] = acc * scales[o];
            } else {
                /* kernels.rs:46-81: lo then hi per byte, odd tail last */
                int64_t rb = (in_dim + 1) / 2, pairs = in_dim / 2;
                const uint8_t *row = (const uint8_t *)payload + o * rb;
                for (int64_t p = 0; p < pairs; p++) {
                    uint8_t b = row[p];
                    int8_t lo = (int8_t)((int8_t)(b << 4) >> 4);
                    int8_t hi = (int8_t)((int8_t)b >> 4);
                    acc += xs[2 * p] * (float)lo;
                    acc += xs[2 * p + 1] * (float)hi;
                }
                if (in_dim % 2 == 1) {
                    uint8_t b = row[pairs];
                    int8_t lo = (int8_t)((int8_t)(b << 4) >> 4);
                    acc += xs[in_dim - 1] * (float)lo;
                }
                os[o] = acc * scales[o];
            }
        }
    }
}

void uto_matvec_rows(int fmt, const void *payload, const float *scales,
                     int64_t out_dim, int64_t in_dim, int64_t row0,
                     int64_t nrows, const float *x, float *out) {
    (void)out_dim;
    for (int64_t j = 0; j < nrows; j++) {
        float acc = 0.0f;
        if (fmt == UTO_F32) {
            const float *r = (const float *)payload + (row0 + j) * in_dim;
            for (int64_t i = 0; i < in_dim; i++) acc += x[i] * r[i];
            out[j] = acc;
        } else if (fmt == UTO_INT8) {
            const int8_t *r = (const int8_t *)payload + (row0 + j) * in_dim;
            for (int64_t i = 0; i < in_dim; i++) acc += x[i] * (float)r[i];
            out[j] = acc * scales[row0 + j];
        } else {
            const uint8_t *r = (const uint8_t *)payload + (row0 + j) * ((in_dim + 1) / 2);
            for (int64_t i = 0; i < in_dim; i++) acc += x[i] * (float)uto_unpack_i4(r, i);
            out[j] = acc * scales[row0 + j];
        }
    }
}

/* ==================================================================== math */
void uto_rmsnorm(float *out, const float *x, const float *w, int64_t n, float eps) {
    /* lib.rs:91-100: mean of squares in f64, the rest in f32. */
    double ms = 0.0;
    for (int64_t i = 0; i < n; i++) ms += (double)x[i] * (double)x[i];
    ms /= (double)n;
    float r = 1.0f / sqrtf((float)ms + eps);
    for (int64_t i = 0; i < n; i++) out[i] = x[i] * r * w[i];
}

void uto_softmax(float *x, int64_t n) {
    /* lib.rs:103-114 */
    float m = -INFINITY;
    for (int64_t i = 0; i < n; i++) m = fmaxf(m, x[i]);
    float sum = 0.0f;
    for (int64_t i = 0; i < n; i++) {
        x[i] = expf(x[i] - m);
        sum += x[i];
    }
    for (int64_t i = 0; i < n; i++) x[i] /= sum;
}

float uto_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
float uto_silu(float x) { return x / (1.0f + expf(-x)); }

void uto_rope_interleave(float *v, int64_t pos, int64_t dim, float theta) {
    /* attention.rs:106-118 */
    int64_t half = dim / 2;
    float *in = (float *)xcalloc((size_t)dim, 4);
    memcpy(in, v, (size_t)dim * 4);
    for (int64_t j = 0; j < half; j++) {
        float inv = powf(theta, -2.0f * (float)j / (float)dim);
        float ang = (float)pos * inv;
        float sn = sinf(ang), cs = cosf(ang);
        float a = in[2 * j], b = in[2 * j + 1];
        v[j] = a * cs - b * sn;
        v[half + j] = b * cs + a * sn;
    }
    free(in);
}

int64_t uto_argmax(const float *v, int64_t n) {
    /* sample.rs:353-361: first maximum; NaN never wins a `>` compare. */
    int64_t best = 0;
    for (int64_t i = 0; i < n; i++)
        if (v[i] > v[best]) best = i;
    return best;
}

/* topk_indices: a bounded min-heap over (value, index) where "worse" means a
 * smaller value or, on equal values, a larger index (router.rs:51-163). */
typedef struct { float val; int64_t idx; } heap_node;

static int is_worse(const heap_node *a, const heap_node *b) {
    if (a->val < b->val) return 1;
    if (a->val > b->val) return 0;
    return a->idx > b->idx;
}

static void heap_swap(heap_node *h, int64_t i, int64_t j) {
    heap_node t = h[i]; h[i] = h[j]; h[j] = t;
}

static void sift_up(heap_node *h, int64_t i) {
    while (i > 0) {
        int64_t parent = (i - 1) / 2;
        if (is_worse(&h[i], &h[parent])) { heap_swap(h, i, parent); i = parent; }
        else break;
    }
}

static void sift_down(heap_node *h, int64_t i, int64_t len) {
    for (;;) {
        int64_t l = 2 * i + 1, r = 2 * i + 2, worst = i;
        if (l < len && is_worse(&h[l], &h[worst])) worst = l;
        if (r < len && is_worse(&h[r], &h[worst])) worst = r;
        if (worst == i) break;
        heap_swap(h, i, worst);
        i = worst;
    }
}

int64_t uto_topk_indices(const float *v, int64_t n, int64_t k, int64_t *out) {
    int64_t k_eff = k < n ? k : n;
    if (k_eff <= 0) return 0;
    if (k_eff == 1) {
        int64_t best = 0;
        for (int64_t i = 1; i < n; i++)
            if (v[i] > v[best]) best = i;
        out[0] = best;
        return 1;
    }
    heap_node *h = (heap_node *)xcalloc((size_t)k_eff, sizeof(heap_node));
    for (int64_t i = 0; i < k_eff; i++) {
        h[i].val = v[i]; h[i].idx = i;
        sift_up(h, i);
    }
    for (int64_t i = k_eff; i < n; i++) {
        heap_node cand = {v[i], i};
        if (is_worse(&h[0], &cand)) { h[0] = cand; sift_down(h, 0, k_eff); }
    }
    for (int64_t step = k_eff - 1; step >= 1; step--) {
        heap_swap(h, 0, step);
        sift_down(h, 0, step);
    }
    for (int64_t i = 0; i < k_eff; i++) out[i] = h[i].idx;
    free(h);
    return k_eff;
}

void uto_route(const float *logits, const float *bias, int64_t e, int64_t top_k,
               int64_t n_group, int64_t topk_group, int norm_topk_prob,
               float routed_scaling_factor, int64_t *ids, float *weights) {
    /* adapters/undertow-deepseek-moe/src/router.rs:58-113 */
    float *scores = (float *)xcalloc((size_t)e, 4);
    float *corr = (float *)xcalloc((size_t)e, 4);
    unsigned char *eligible = (unsigned char *)xcalloc((size_t)e, 1);
    for (int64_t i = 0; i < e; i++) {
        scores[i] = uto_sigmoid(logits[i]);
        corr[i] = scores[i];
        if (bias) corr[i] += bias[i];
        eligible[i] = 1;
    }
    if (n_group > 1 && topk_group < n_group) {
        int64_t gs = e / n_group;
        float *gscore = (float *)xcalloc((size_t)n_group, 4);
        int64_t two[2];
        for (int64_t g = 0; g < n_group; g++) {
            int64_t c = uto_topk_indices(corr + g * gs, gs, 2, two);
            float s = 0.0f; /* iterator sum over the chosen pair, in order */
            for (int64_t j = 0; j < c; j++) s += corr[g * gs + two[j]];
            gscore[g] = s;
        }
        int64_t *tg = (int64_t *)xcalloc((size_t)topk_group, 8);
        int64_t ng = uto_topk_indices(gscore, n_group, topk_group, tg);
        memset(eligible, 0, (size_t)e);
        for (int64_t j = 0; j < ng; j++)
            memset(eligible + tg[j] * gs, 1, (size_t)gs);
        free(tg);
        free(gscore);
    }
    float *masked = (float *)xcalloc((size_t)e, 4);
    for (int64_t i = 0; i < e; i++) masked[i] = eligible[i] ? corr[i] : -INFINITY;
    int64_t kk = uto_topk_indices(masked, e, top_k, ids);
    float *w = (float *)xcalloc((size_t)(kk ? kk : 1), 4);
    for (int64_t j = 0; j < kk; j++) w[j] = scores[ids[j]];
    if (norm_topk_prob) {
        float denom = 0.0f;
        for (int64_t j = 0; j < kk; j++) denom += w[j];
        denom += 1e-20f;
        for (int64_t j = 0; j < kk; j++) w[j] /= denom;
    }
    for (int64_t j = 0; j < kk; j++) weights[j] = w[j] * routed_scaling_factor;
    free(w); free(masked); free(eligible); free(corr); free(scores);
}

/* ============================================================= expert FFN */
void uto_mlp_forward_add(int fmt, int64_t hidden, int64_t inter,
                         const void *gp, const float *gs, const void *upp,
                         const float *us, const void *dp, const float *ds,
                         const float *x, int64_t seq, float *out) {
    /* model.rs:43-58 */
    float *g = (float *)xcalloc((size_t)(seq * inter), 4);
    float *u = (float *)xcalloc((size_t)(seq * inter), 4);
    float *d = (float *)xcalloc((size_t)(seq * hidden), 4);
    uto_matmul(fmt, gp, gs, inter, hidden, x, seq, g);
    uto_matmul(fmt, upp, us, inter, hidden, x, seq, u);
    for (int64_t i = 0; i < seq * inter; i++) g[i] = uto_silu(g[i]) * u[i];
    uto_matmul(fmt, dp, ds, hidden, inter, g, seq, d);
    for (int64_t i = 0; i < seq * hidden; i++) out[i] += d[i];
    free(g); free(u); free(d);
}

void uto_moe_experts(int fmt, int64_t hidden, int64_t inter,
                     const uint8_t *gate_payload, const float *gate_scales,
                     const uint8_t *up_payload, const float *up_scales,
                     const uint8_t *down_payload, const float *down_scales,
                     int64_t M, int64_t top_k, const int64_t *ids,
                     const float *weights, const float *x, float *out) {
    /* Each (row, choice) computed per row: the reference groups rows by
     * expert, but matmul numerics are per-row independent (qtensor.rs:274-280)
     * so the per-row evaluation is the same arithmetic. */
    int64_t gbytes = uto_payload_bytes(fmt, inter, hidden);
    int64_t dbytes = uto_payload_bytes(fmt, hidden, inter);
    float *g = (float *)xcalloc((size_t)inter, 4);
    float *u = (float *)xcalloc((size_t)inter, 4);
    float *d = (float *)xcalloc((size_t)hidden, 4);
    memset(out, 0, (size_t)(M * hidden) * 4);
    for (int64_t s = 0; s < M; s++) {
        const float *xs = x + s * hidden;
        for (int64_t c = 0; c < top_k; c++) {
            int64_t e = ids[s * top_k + c];
            uto_matmul(fmt, gate_payload + e * gbytes, gate_scales + e * inter,
                       inter, hidden, xs, 1, g);
            uto_matmul(fmt, up_payload + e * gbytes, up_scales + e * inter,
                       inter, hidden, xs, 1, u);
            for (int64_t i = 0; i < inter; i++) g[i] = uto_silu(g[i]) * u[i];
            uto_matmul(fmt, down_payload + e * dbytes, down_scales + e * hidden,
                       hidden, inter, g, 1, d);
            float w = weights[s * top_k + c];
            float *os = out + s * hidden;
            for (int64_t i = 0; i < hidden; i++) os[i] += w * d[i];
        }
    }
    free(g); free(u); free(d);
}

/* ================================================================ MLA core */
void uto_mla_attend(const float *qabs, const float *q_rope, const float *latent,
                    const float *krot, int64_t R, int64_t H, int64_t L,
                    int64_t P, int64_t pos_base, float scale, float *clat) {
    /* attention.rs:214-234; the (row, head) pairs are independent (the
     * reference runs them as rayon tasks, attention.rs:202), each in its
     * sequential order */
    int64_t nmax = pos_base + R;
#pragma omp parallel for collapse(2) schedule(dynamic) if (R * H * nmax >= (1 << 14))
    for (int64_t s = 0; s < R; s++) {
        for (int64_t h = 0; h < H; h++) {
            float *scores = (float *)xcalloc((size_t)nmax, 4);
            int64_t n_ctx = pos_base + s + 1;
            const float *qa = qabs + (s * H + h) * L;
            const float *qr = q_rope + (s * H + h) * P;
            for (int64_t t = 0; t < n_ctx; t++) {
                const float *lat = latent + t * L;
                const float *kr = krot + t * P;
                float a = 0.0f;
                for (int64_t i = 0; i < L; i++) a += qa[i] * lat[i];
                for (int64_t i = 0; i < P; i++) a += qr[i] * kr[i];
                scores[t] = a * scale;
            }
            uto_softmax(scores, n_ctx);
            float *cl = clat + (s * H + h) * L;
            for (int64_t i = 0; i < L; i++) cl[i] = 0.0f;
            for (int64_t t = 0; t < n_ctx; t++) {
                const float *lat = latent + t * L;
                float a = scores[t];
                for (int64_t i = 0; i < L; i++) cl[i] += a * lat[i];
            }
            free(scores);
        }
    }
}

/* ============================================================ checkpoint */
typedef struct {
    char name[128];
    int32_t ndim;
    int64_t shape[2];
    int32_t fmt;       /* UTO_F32 / UTO_INT8 / UTO_INT4 */
    void *payload;     /* f32 data, int8 codes or packed int4 */
    int64_t nbytes;
    float *scales;     /* NULL for f32 */
} uto_tensor;

struct uto_ckpt {
    uto_tensor *t;
    int64_t n, cap;
};

void uto_spec_default(uto_spec *s) {
    /* OracleSpec::default (oracle.rs:46-75) */
    memset(s, 0, sizeof(*s));
    s->seed = 20260712;
    s->vocab_size = 256;
    s->hidden_size = 64;
    s->intermediate_size = 128;
    s->moe_intermediate_size = 32;
    s->num_hidden_layers = 4;
    s->first_k_dense_replace = 1;
    s->num_attention_heads = 4;
    s->n_routed_experts = 16;
    s->num_experts_per_tok = 4;
    s->n_shared_experts = 1;
    s->n_group = 4;
    s->topk_group = 2;
    s->norm_topk_prob = 1;
    s->routed_scaling_factor = 2.5f;
    s->q_lora_rank = 32;
    s->kv_lora_rank = 16;
    s->qk_nope_head_dim = 16;
    s->qk_rope_head_dim = 8;
    s->v_head_dim = 16;
    s->rms_norm_eps = 1e-6f;
    s->rope_theta = 10000.0f;
    s->init_std = 0.05f;
    s->mtp = 1;
    s->max_position_embeddings = 4096;
}

static uto_tensor *ck_push_empty(uto_ckpt *c, const char *name, int ndim, int64_t d0,
                                 int64_t d1) {
    if (c->n == c->cap) {
        c->cap = c->cap ? c->cap * 2 : 256;
        c->t = (uto_tensor *)realloc(c->t, (size_t)c->cap * sizeof(uto_tensor));
        if (!c->t) abort();
    }
    uto_tensor *t = &c->t[c->n++];
    memset(t, 0, sizeof(*t));
    snprintf(t->name, sizeof(t->name), "%s", name);
    t->ndim = ndim;
    t->shape[0] = d0;
    t->shape[1] = ndim == 2 ? d1 : 1;
    t->fmt = UTO_F32;
    return t;
}

static uto_tensor *ck_push(uto_ckpt *c, const char *name, int ndim, int64_t d0,
                           int64_t d1) {
    if (c->n == c->cap) {
        c->cap = c->cap ? c->cap * 2 : 256;
        c->t = (uto_tensor *)realloc(c->t, (size_t)c->cap * sizeof(uto_tensor));
        if (!c->t) abort();
    }
    uto_tensor *t = &c->t[c->n++];
    memset(t, 0, sizeof(*t));
    snprintf(t->name, sizeof(t->name), "%s", name);
    t->ndim = ndim;
    t->shape[0] = d0;
    t->shape[1] = ndim == 2 ? d1 : 1;
    t->fmt = UTO_F32;
    int64_t n = d0 * (ndim == 2 ? d1 : 1);
    t->payload = xcalloc((size_t)n, 4);
    t->nbytes = n * 4;
    return t;
}

typedef struct { uto_ckpt *c; uto_pcg32 rng; float std; int skip_mats; } gen_state;

static void g_mat(gen_state *g, const char *name, int64_t d0, int64_t d1) {
    /* Gen::mat (oracle.rs:126-132): normal() * std, row-major.  skip_mats:
     * leave the matrix for uto_ckpt_synthesize to fill. */
    if (g->skip_mats) {
        ck_push_empty(g->c, name, 2, d0, d1);
        return;
    }
    uto_tensor *t = ck_push(g->c, name, 2, d0, d1);
    float *d = (float *)t->payload;
    for (int64_t i = 0; i < d0 * d1; i++) d[i] = uto_pcg32_normal(&g->rng) * g->std;
}

static void g_norm(gen_state *g, const char *name, int64_t n) {
    /* Gen::norm (oracle.rs:136-141): 1 + (uniform - 0.5) * 0.2 */
    uto_tensor *t = ck_push(g->c, name, 1, n, 1);
    float *d = (float *)t->payload;
    for (int64_t i = 0; i < n; i++) d[i] = 1.0f + (uto_pcg32_uniform(&g->rng) - 0.5f) * 0.2f;
}

static void g_bias(gen_state *g, const char *name, int64_t e) {
    /* oracle.rs:205-209: -0.1 + 0.2 * i / max(e-1, 1) */
    uto_tensor *t = ck_push(g->c, name, 1, e, 1);
    float *d = (float *)t->payload;
    float den = (float)(e - 1 > 1 ? e - 1 : 1);
    for (int64_t i = 0; i < e; i++) d[i] = -0.1f + 0.2f * (float)i / den;
}

static void g_layer_attn(gen_state *g, const uto_spec *s, int64_t li) {
    char nm[160];
    int64_t hd = s->hidden_size, heads = s->num_attention_heads;
    int64_t qh = s->qk_nope_head_dim + s->qk_rope_head_dim;
    snprintf(nm, sizeof nm, "model.layers.%lld.input_layernorm.weight", (long long)li); g_norm(g, nm, hd);
    snprintf(nm, sizeof nm, "model.layers.%lld.post_attention_layernorm.weight", (long long)li); g_norm(g, nm, hd);
    snprintf(nm, sizeof nm, "model.layers.%lld.self_attn.q_a_proj.weight", (long long)li); g_mat(g, nm, s->q_lora_rank, hd);
    snprintf(nm, sizeof nm, "model.layers.%lld.self_attn.q_a_layernorm.weight", (long long)li); g_norm(g, nm, s->q_lora_rank);
    snprintf(nm, sizeof nm, "model.layers.%lld.self_attn.q_b_proj.weight", (long long)li); g_mat(g, nm, heads * qh, s->q_lora_rank);
    snprintf(nm, sizeof nm, "model.layers.%lld.self_attn.kv_a_proj_with_mqa.weight", (long long)li);
    g_mat(g, nm, s->kv_lora_rank + s->qk_rope_head_dim, hd);
    snprintf(nm, sizeof nm, "model.layers.%lld.self_attn.kv_a_layernorm.weight", (long long)li); g_norm(g, nm, s->kv_lora_rank);
    snprintf(nm, sizeof nm, "model.layers.%lld.self_attn.kv_b_proj.weight", (long long)li);
    g_mat(g, nm, heads * (s->qk_nope_head_dim + s->v_head_dim), s->kv_lora_rank);
    snprintf(nm, sizeof nm, "model.layers.%lld.self_attn.o_proj.weight", (long long)li); g_mat(g, nm, hd, heads * s->v_head_dim);
}

static void g_moe(gen_state *g, const uto_spec *s, int64_t li) {
    char nm[160];
    int64_t hd = s->hidden_size, e = s->n_routed_experts;
    snprintf(nm, sizeof nm, "model.layers.%lld.mlp.gate.weight", (long long)li); g_mat(g, nm, e, hd);
    snprintf(nm, sizeof nm, "model.layers.%lld.mlp.gate.e_score_correction_bias", (long long)li); g_bias(g, nm, e);
    for (int64_t ei = 0; ei < e; ei++) {
        snprintf(nm, sizeof nm, "model.layers.%lld.mlp.experts.%lld.gate_proj.weight", (long long)li, (long long)ei);
        g_mat(g, nm, s->moe_intermediate_size, hd);
        snprintf(nm, sizeof nm, "model.layers.%lld.mlp.experts.%lld.up_proj.weight", (long long)li, (long long)ei);
        g_mat(g, nm, s->moe_intermediate_size, hd);
        snprintf(nm, sizeof nm, "model.layers.%lld.mlp.experts.%lld.down_proj.weight", (long long)li, (long long)ei);
        g_mat(g, nm, hd, s->moe_intermediate_size);
    }
    if (s->n_shared_experts > 0) {
        int64_t si = s->n_shared_experts * s->moe_intermediate_size;
        snprintf(nm, sizeof nm, "model.layers.%lld.mlp.shared_experts.gate_proj.weight", (long long)li); g_mat(g, nm, si, hd);
        snprintf(nm, sizeof nm, "model.layers.%lld.mlp.shared_experts.up_proj.weight", (long long)li); g_mat(g, nm, si, hd);
        snprintf(nm, sizeof nm, "model.layers.%lld.mlp.shared_experts.down_proj.weight", (long long)li); g_mat(g, nm, hd, si);
    }
}

static uto_ckpt *generate(const uto_spec *s, int skip_mats) {
    /* generate_oracle (oracle.rs:150-310), tensor order preserved. */
    uto_ckpt *c = (uto_ckpt *)xcalloc(1, sizeof(uto_ckpt));
    gen_state g;
    g.c = c;
    g.std = s->init_std;
    g.skip_mats = skip_mats;
    uto_pcg32_init(&g.rng, s->seed, 54);
    char nm[160];
    int64_t hd = s->hidden_size;
    g_mat(&g, "model.embed_tokens.weight", s->vocab_size, hd);
    for (int64_t li = 0; li < s->num_hidden_layers; li++) {
        g_layer_attn(&g, s, li);
        if (li < s->first_k_dense_replace) {
            snprintf(nm, sizeof nm, "model.layers.%lld.mlp.gate_proj.weight", (long long)li); g_mat(&g, nm, s->intermediate_size, hd);
            snprintf(nm, sizeof nm, "model.layers.%lld.mlp.up_proj.weight", (long long)li); g_mat(&g, nm, s->intermediate_size, hd);
            snprintf(nm, sizeof nm, "model.layers.%lld.mlp.down_proj.weight", (long long)li); g_mat(&g, nm, hd, s->intermediate_size);
        } else {
            g_moe(&g, s, li);
        }
    }
    g_norm(&g, "model.norm.weight", hd);
    g_mat(&g, "lm_head.weight", s->vocab_size, hd);
    if (s->mtp) {
        int64_t li = s->num_hidden_layers;
        g_layer_attn(&g, s, li);
        g_moe(&g, s, li);
        snprintf(nm, sizeof nm, "model.layers.%lld.enorm.weight", (long long)li); g_norm(&g, nm, hd);
        snprintf(nm, sizeof nm, "model.layers.%lld.hnorm.weight", (long long)li); g_norm(&g, nm, hd);
        snprintf(nm, sizeof nm, "model.layers.%lld.eh_proj.weight", (long long)li); g_mat(&g, nm, hd, 2 * hd);
        snprintf(nm, sizeof nm, "model.layers.%lld.shared_head.norm.weight", (long long)li); g_norm(&g, nm, hd);
        snprintf(nm, sizeof nm, "model.layers.%lld.shared_head.head.weight", (long long)li); g_mat(&g, nm, s->vocab_size, hd);
    }
    return c;
}

uto_ckpt *uto_generate(const uto_spec *s) { return generate(s, 0); }

void uto_ckpt_free(uto_ckpt *c) {
    if (!c) return;
    for (int64_t i = 0; i < c->n; i++) { free(c->t[i].payload); free(c->t[i].scales); }
    free(c->t);
    free(c);
}

static int cmp_idx_by_name(const void *a, const void *b, void *ctx) {
    const uto_ckpt *c = (const uto_ckpt *)ctx;
    return strcmp(c->t[*(const int64_t *)a].name, c->t[*(const int64_t *)b].name);
}

/* Plain insertion sort with a context (qsort_r portability is not worth it). */
static void sort_idx(int64_t *idx, int64_t n, const uto_ckpt *c) {
    for (int64_t i = 1; i < n; i++) {
        int64_t v = idx[i], j = i - 1;
        while (j >= 0 && cmp_idx_by_name(&idx[j], &v, (void *)c) > 0) { idx[j + 1] = idx[j]; j--; }
        idx[j + 1] = v;
    }
}

typedef struct { char *p; int64_t n, cap; } sbuf;
static void sb_put(sbuf *b, const char *s, int64_t n) {
    if (b->n + n + 1 > b->cap) {
        b->cap = (b->n + n + 1) * 2;
        b->p = (char *)realloc(b->p, (size_t)b->cap);
        if (!b->p) abort();
    }
    memcpy(b->p + b->n, s, (size_t)n);
    b->n += n;
}
static void sb_str(sbuf *b, const char *s) { sb_put(b, s, (int64_t)strlen(s)); }

int64_t uto_ckpt_safetensors(const uto_ckpt *c, uint8_t *buf, int64_t cap) {
    /* writer.rs:73-110 with TensorEntry::f32 / from_qtensor entries
     * (writer.rs:16-64): serde_json map = keys in byte order, compact,
     * header padded with spaces to a multiple of 8, data in entry order. */
    int64_t nent = 0;
    for (int64_t i = 0; i < c->n; i++) nent += c->t[i].fmt == UTO_F32 ? 1 : 2;
    typedef struct { char name[160]; const char *dtype; int nd; int64_t sh[2]; const void *data; int64_t nbytes; } ent;
    ent *e = (ent *)xcalloc((size_t)nent, sizeof(ent));
    int64_t k = 0;
    for (int64_t i = 0; i < c->n; i++) {
        const uto_tensor *t = &c->t[i];
        snprintf(e[k].name, sizeof e[k].name, "%s", t->name);
        e[k].data = t->payload;
        e[k].nbytes = t->nbytes;
        if (t->fmt == UTO_F32) {
            e[k].dtype = "F32"; e[k].nd = t->ndim; e[k].sh[0] = t->shape[0]; e[k].sh[1] = t->shape[1];
            k++;
        } else {
            e[k].dtype = "U8"; e[k].nd = 2; e[k].sh[0] = t->shape[0];
            e[k].sh[1] = t->fmt == UTO_INT8 ? t->shape[1] : (t->shape[1] + 1) / 2;
            k++;
            snprintf(e[k].name, sizeof e[k].name, "%s.scales", t->name);
            e[k].dtype = "F32"; e[k].nd = 1; e[k].sh[0] = t->shape[0];
            e[k].data = t->scales; e[k].nbytes = t->shape[0] * 4;
            k++;
        }
    }
    int64_t *off = (int64_t *)xcalloc((size_t)nent, 8);
    int64_t o = 0;
    for (int64_t i = 0; i < nent; i++) { off[i] = o; o += e[i].nbytes; }
    /* sort entry indices by name for the header */
    int64_t *idx = (int64_t *)xcalloc((size_t)nent, 8);
    for (int64_t i = 0; i < nent; i++) idx[i] = i;
    for (int64_t i = 1; i < nent; i++) {
        int64_t v = idx[i], j = i - 1;
        while (j >= 0 && strcmp(e[idx[j]].name, e[v].name) > 0) { idx[j + 1] = idx[j]; j--; }
        idx[j + 1] = v;
    }
    sbuf h = {0};
    char tmp[512];
    sb_str(&h, "{");
    for (int64_t q = 0; q < nent; q++) {
        const ent *x = &e[idx[q]];
        if (q) sb_str(&h, ",");
        if (x->nd == 2)
            snprintf(tmp, sizeof tmp, "\"%s\":{\"data_offsets\":[%lld,%lld],\"dtype\":\"%s\",\"shape\":[%lld,%lld]}",
                     x->name, (long long)off[idx[q]], (long long)(off[idx[q]] + x->nbytes), x->dtype,
                     (long long)x->sh[0], (long long)x->sh[1]);
        else
            snprintf(tmp, sizeof tmp, "\"%s\":{\"data_offsets\":[%lld,%lld],\"dtype\":\"%s\",\"shape\":[%lld]}",
                     x->name, (long long)off[idx[q]], (long long)(off[idx[q]] + x->nbytes), x->dtype,
                     (long long)x->sh[0]);
        sb_str(&h, tmp);
    }
    sb_str(&h, "}");
    while (h.n % 8) sb_str(&h, " ");
    int64_t total = 8 + h.n + o;
    if (buf && cap >= total) {
        uint64_t hl = (uint64_t)h.n;
        for (int i = 0; i < 8; i++) buf[i] = (uint8_t)(hl >> (8 * i));
        memcpy(buf + 8, h.p, (size_t)h.n);
        for (int64_t i = 0; i < nent; i++)
            memcpy(buf + 8 + h.n + off[i], e[i].data, (size_t)e[i].nbytes);
    }
    free(h.p); free(idx); free(off); free(e);
    (void)sort_idx;
    return total;
}

/* classify_tensor (adapters/undertow-deepseek-moe/src/naming.rs:28-73):
 * 0 = KeepF32, 1 = Dense, 2 = Expert. */
static int classify(const char *name) {
    static const char *dense_suffixes[] = {
        ".self_attn.q_proj.weight", ".self_attn.q_a_proj.weight", ".self_attn.q_b_proj.weight",
        ".self_attn.kv_a_proj_with_mqa.weight", ".self_attn.kv_b_proj.weight", ".self_attn.o_proj.weight",
        ".mlp.gate_proj.weight", ".mlp.up_proj.weight", ".mlp.down_proj.weight",
        ".mlp.shared_experts.gate_proj.weight", ".mlp.shared_experts.up_proj.weight",
        ".mlp.shared_experts.down_proj.weight", ".eh_proj.weight", ".embed_tokens.weight",
        ".shared_head.head.weight"};
    const char *pre = "model.layers.";
    size_t n = strlen(name);
    if (strncmp(name, pre, strlen(pre)) == 0) {
        const char *rest = name + strlen(pre);
        const char *dot = strchr(rest, '.');
        if (dot && dot > rest) {
            int digits = 1;
            for (const char *p = rest; p < dot; p++) if (*p < '0' || *p > '9') digits = 0;
            const char *tail = dot + 1;
            size_t tl = strlen(tail);
            if (digits && strncmp(tail, "mlp.experts.", 12) == 0 && tl >= 7 &&
                strcmp(tail + tl - 7, ".weight") == 0)
                return 2;
        }
    }
    if (strcmp(name, "lm_head.weight") == 0) return 1;
    for (size_t i = 0; i < sizeof dense_suffixes / sizeof dense_suffixes[0]; i++) {
        size_t sl = strlen(dense_suffixes[i]);
        if (n >= sl && strcmp(name + n - sl, dense_suffixes[i]) == 0) return 1;
    }
    return 0;
}

int uto_ckpt_convert(uto_ckpt *c, int expert_fmt, int dense_fmt) {
    for (int64_t i = 0; i < c->n; i++) {
        uto_tensor *t = &c->t[i];
        if (t->ndim != 2 || t->fmt != UTO_F32) continue;
        int d = classify(t->name);
        int fmt = d == 2 ? expert_fmt : (d == 1 ? dense_fmt : UTO_F32);
        if (fmt == UTO_F32) continue;
        int64_t o = t->shape[0], in = t->shape[1];
        int64_t nb = uto_payload_bytes(fmt, o, in);
        void *p = xcalloc((size_t)nb, 1);
        float *sc = (float *)xcalloc((size_t)o, 4);
        if (uto_quantize(fmt, (const float *)t->payload, o, in, p, sc) != 0) {
            free(p); free(sc);
            return -1;
        }
        free(t->payload);
        t->payload = p;
        t->nbytes = nb;
        t->scales = sc;
        t->fmt = fmt;
    }
    return 0;
}

int64_t uto_ckpt_count(const uto_ckpt *c) { return c->n; }

int uto_ckpt_info(const uto_ckpt *c, int64_t i, char *name, int64_t name_cap,
                  int32_t *fmt, int64_t *shape, int32_t *ndim) {
    if (i < 0 || i >= c->n) return -1;
    const uto_tensor *t = &c->t[i];
    if (name && name_cap > 0) snprintf(name, (size_t)name_cap, "%s", t->name);
    if (fmt) *fmt = t->fmt;
    if (shape) { shape[0] = t->shape[0]; shape[1] = t->shape[1]; }
    if (ndim) *ndim = t->ndim;
    return 0;
}

const void *uto_ckpt_payload(const uto_ckpt *c, int64_t i, int64_t *nbytes) {
    if (i < 0 || i >= c->n) return NULL;
    if (nbytes) *nbytes = c->t[i].nbytes;
    return c->t[i].payload;
}

const float *uto_ckpt_scales(const uto_ckpt *c, int64_t i) {
    if (i < 0 || i >= c->n) return NULL;
    return c->t[i].scales;
}

uto_ckpt *uto_ckpt_new(void) { return (uto_ckpt *)xcalloc(1, sizeof(uto_ckpt)); }

int uto_ckpt_add(uto_ckpt *c, const char *name, int32_t fmt, int32_t ndim, int64_t d0, int64_t d1,
                 const void *payload, int64_t nbytes, const float *scales) {
    if (ndim != 1 && ndim != 2) return -1;
    if (ndim == 1 && fmt != UTO_F32) return -1;
    if (nbytes != uto_payload_bytes(fmt, d0, ndim == 2 ? d1 : 1)) return -1;
    if (fmt != UTO_F32 && !scales) return -1;
    uto_tensor *t = ck_push(c, name, ndim, d0, d1);
    free(t->payload);
    t->payload = xcalloc((size_t)nbytes, 1);
    memcpy(t->payload, payload, (size_t)nbytes);
    t->nbytes = nbytes;
    t->fmt = fmt;
    if (fmt != UTO_F32) {
        t->scales = (float *)xcalloc((size_t)d0, 4);
        memcpy(t->scales, scales, (size_t)d0 * 4);
    }
    return 0;
}

/* ----------------------------------------------------- synthetic weights */
/* Test inputs at DeepSeek-V3 width, where generate_oracle's Irwin-Hall
 * stream would take minutes: each element is a pure function of (seed,
 * tensor ordinal, element index) through splitmix64, so rows fill in
 * parallel.  The distributions are the benchmark's: quantized codes uniform
 * over the format's range, per-row scales |N(0,std)|/qmax, f32 matrices
 * N(0,std), norms 1 +- 0.1, the bias ramp of oracle.rs:205-209. */
static uint64_t splitmix(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

static float syn_u01(uint64_t key, uint64_t i) {
    return (float)((splitmix(key ^ splitmix(i)) >> 40) + 0.5) * (1.0f / 16777216.0f);
}

static float syn_normal(uint64_t key, uint64_t i) {
    /* Box-Muller over two uniforms of the element's stream */
    float u1 = syn_u01(key, 2 * i), u2 = syn_u01(key, 2 * i + 1);
    return sqrtf(-2.0f * logf(u1)) * cosf(6.2831853f * u2);
}

/* Buffers of many megabytes on transparent huge pages where the kernel
 * offers them (a fault per 2 MiB instead of per 4 KiB); every byte is
 * written by the caller. */
static void *big_alloc(size_t n) {
    const size_t huge = (size_t)2 << 20;
    if (n < huge) return xcalloc(n, 1);
    size_t sz = (n + huge - 1) / huge * huge;
    void *p = aligned_alloc(huge, sz);
    if (!p) { fprintf(stderr, "ut_oracle: out of memory\n"); abort(); }
#ifdef MADV_HUGEPAGE
    madvise(p, sz, MADV_HUGEPAGE);
#endif
    return p;
}

static void syn_tensor(uto_tensor *t, uint64_t key, int fmt, float std) {
    int64_t o = t->shape[0], in = t->ndim == 2 ? t->shape[1] : 1;
    if (fmt == UTO_F32) {
        free(t->payload);
        t->nbytes = o * in * 4;
        t->payload = big_alloc((size_t)t->nbytes);
        float *d = (float *)t->payload;
#pragma omp parallel for schedule(static)
        for (int64_t r = 0; r < o; r++)
            for (int64_t i = 0; i < in; i++) d[r * in + i] = syn_normal(key, (uint64_t)(r * in + i)) * std;
        return;
    }
    int64_t nb = uto_payload_bytes(fmt, o, in), rb = nb / o;
    uint8_t *p = (uint8_t *)big_alloc((size_t)nb);
    float *sc = (float *)xcalloc((size_t)o, 4);
    float qmax = fmt == UTO_INT4 ? 7.0f : 127.0f;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < o; r++) {
        uint8_t *row = p + r * rb;
        for (int64_t b = 0; b < rb; b += 8) {
            uint64_t v = splitmix(key ^ splitmix((uint64_t)(r * rb + b) | (1ull << 62)));
            for (int64_t j = 0; j < 8 && b + j < rb; j++) {
                uint8_t byte = (uint8_t)(v >> (8 * j));
                if (fmt == UTO_INT8) byte = (uint8_t)(int8_t)((int)(byte % 255u) - 127);
                row[b + j] = byte;
            }
        }
        if (fmt == UTO_INT4 && in % 2 == 1) row[rb - 1] &= 0x0F;
        sc[r] = fabsf(syn_normal(key ^ 0x5ca1e5ull, (uint64_t)r)) * std / qmax;
    }
    free(t->payload);
    t->payload = p;
    t->nbytes = nb;
    t->scales = sc;
    t->fmt = fmt;
}

uto_ckpt *uto_ckpt_synthesize(const uto_spec *s, uint64_t seed, float std, int expert_fmt,
                              int dense_fmt) {
    /* uto_generate's tensor list (norms and bias as generated), every
     * matrix filled by syn_tensor in the format the converter would give it
     * (classify_tensor: experts expert_fmt, dense dense_fmt, router gate f32) */
    uto_ckpt *c = generate(s, 1);
    for (int64_t i = 0; i < c->n; i++) {
        uto_tensor *t = &c->t[i];
        if (t->ndim != 2) continue;
        int d = classify(t->name);
        int fmt = d == 2 ? expert_fmt : (d == 1 ? dense_fmt : UTO_F32);
        syn_tensor(t, splitmix(seed ^ splitmix((uint64_t)i + 1)), fmt, std);
    }
    return c;
}

/* ================================================================= model */
typedef struct { int32_t fmt; int64_t out_dim, in_dim; const void *p; const float *s; } qt;

static void qt_matmul(const qt *w, const float *x, int64_t seq, float *out) {
    uto_matmul(w->fmt, w->p, w->s, w->out_dim, w->in_dim, x, seq, out);
}

typedef struct { qt gate, up, down; } mlp_w;

typedef struct {
    const float *input_norm, *post_norm;
    int lora;
    qt q_a, q_b, q_proj, kv_a, kv_b, o_proj;
    const float *q_a_norm, *kv_a_norm;
    int dense;
    mlp_w mlp;          /* dense FFN */
    const float *gate;  /* router gate [E, H] f32 */
    const float *bias;  /* e_score_correction_bias or NULL */
    int has_shared;
    mlp_w shared;
    mlp_w *experts;     /* [E] */
} layer_w;

struct uto_model {
    uto_spec c;
    qt embed, lm_head;
    const float *final_norm;
    layer_w *layers;
    int has_mtp;
    const float *enorm, *hnorm, *mtp_norm;
    qt eh_proj, mtp_head;
    layer_w mtp_layer;
};

static const uto_tensor *find(const uto_ckpt *c, const char *name) {
    for (int64_t i = 0; i < c->n; i++)
        if (strcmp(c->t[i].name, name) == 0) return &c->t[i];
    return NULL;
}

static int get_qt(const uto_ckpt *c, const char *name, int64_t o, int64_t in, qt *out) {
    const uto_tensor *t = find(c, name);
    if (!t || t->ndim != 2 || t->shape[0] != o || t->shape[1] != in) {
        fprintf(stderr, "ut_oracle: missing or misshapen tensor %s\n", name);
        return -1;
    }
    out->fmt = t->fmt; out->out_dim = o; out->in_dim = in; out->p = t->payload; out->s = t->scales;
    return 0;
}

static const float *get_vec(const uto_ckpt *c, const char *name, int64_t n) {
    const uto_tensor *t = find(c, name);
    if (!t || t->fmt != UTO_F32 || t->shape[0] * (t->ndim == 2 ? t->shape[1] : 1) != n) {
        fprintf(stderr, "ut_oracle: missing or misshapen tensor %s\n", name);
        return NULL;
    }
    return (const float *)t->payload;
}

static int load_layer(const uto_ckpt *c, const uto_spec *s, int64_t li, int dense, layer_w *L) {
    char nm[200];
    int64_t hd = s->hidden_size, heads = s->num_attention_heads;
    int64_t qh = s->qk_nope_head_dim + s->qk_rope_head_dim;
    int rc = 0;
    memset(L, 0, sizeof(*L));
#define P(fmt_) (snprintf(nm, sizeof nm, "model.layers.%lld." fmt_, (long long)li), nm)
    L->input_norm = get_vec(c, P("input_layernorm.weight"), hd);
    L->post_norm = get_vec(c, P("post_attention_layernorm.weight"), hd);
    if (s->q_lora_rank > 0) {
        L->lora = 1;
        rc |= get_qt(c, P("self_attn.q_a_proj.weight"), s->q_lora_rank, hd, &L->q_a);
        L->q_a_norm = get_vec(c, P("self_attn.q_a_layernorm.weight"), s->q_lora_rank);
        rc |= get_qt(c, P("self_attn.q_b_proj.weight"), heads * qh, s->q_lora_rank, &L->q_b);
    } else {
        rc |= get_qt(c, P("self_attn.q_proj.weight"), heads * qh, hd, &L->q_proj);
    }
    rc |= get_qt(c, P("self_attn.kv_a_proj_with_mqa.weight"), s->kv_lora_rank + s->qk_rope_head_dim, hd, &L->kv_a);
    L->kv_a_norm = get_vec(c, P("self_attn.kv_a_layernorm.weight"), s->kv_lora_rank);
    rc |= get_qt(c, P("self_attn.kv_b_proj.weight"), heads * (s->qk_nope_head_dim + s->v_head_dim), s->kv_lora_rank, &L->kv_b);
    rc |= get_qt(c, P("self_attn.o_proj.weight"), hd, heads * s->v_head_dim, &L->o_proj);
    L->dense = dense;
    if (dense) {
        rc |= get_qt(c, P("mlp.gate_proj.weight"), s->intermediate_size, hd, &L->mlp.gate);
        rc |= get_qt(c, P("mlp.up_proj.weight"), s->intermediate_size, hd, &L->mlp.up);
        rc |= get_qt(c, P("mlp.down_proj.weight"), hd, s->intermediate_size, &L->mlp.down);
    } else {
        L->gate = get_vec(c, P("mlp.gate.weight"), s->n_routed_experts * hd);
        L->bias = find(c, P("mlp.gate.e_score_correction_bias")) ? get_vec(c, nm, s->n_routed_experts) : NULL;
        if (s->n_shared_experts > 0) {
            int64_t si = s->n_shared_experts * s->moe_intermediate_size;
            L->has_shared = 1;
            rc |= get_qt(c, P("mlp.shared_experts.gate_proj.weight"), si, hd, &L->shared.gate);
            rc |= get_qt(c, P("mlp.shared_experts.up_proj.weight"), si, hd, &L->shared.up);
            rc |= get_qt(c, P("mlp.shared_experts.down_proj.weight"), hd, si, &L->shared.down);
        }
        L->experts = (mlp_w *)xcalloc((size_t)s->n_routed_experts, sizeof(mlp_w));
        for (int64_t e = 0; e < s->n_routed_experts; e++) {
            snprintf(nm, sizeof nm, "model.layers.%lld.mlp.experts.%lld.gate_proj.weight", (long long)li, (long long)e);
            rc |= get_qt(c, nm, s->moe_intermediate_size, hd, &L->experts[e].gate);
            snprintf(nm, sizeof nm, "model.layers.%lld.mlp.experts.%lld.up_proj.weight", (long long)li, (long long)e);
            rc |= get_qt(c, nm, s->moe_intermediate_size, hd, &L->experts[e].up);
            snprintf(nm, sizeof nm, "model.layers.%lld.mlp.experts.%lld.down_proj.weight", (long long)li, (long long)e);
            rc |= get_qt(c, nm, hd, s->moe_intermediate_size, &L->experts[e].down);
        }
    }
#undef P
    if (!L->input_norm || !L->post_norm || !L->kv_a_norm || (L->lora && !L->q_a_norm) || (!dense && !L->gate))
        rc = -1;
    return rc;
}

uto_model *uto_model_new(const uto_ckpt *c, const uto_spec *s) {
    uto_model *m = (uto_model *)xcalloc(1, sizeof(uto_model));
    m->c = *s;
    int rc = 0;
    int64_t hd = s->hidden_size;
    rc |= get_qt(c, "model.embed_tokens.weight", s->vocab_size, hd, &m->embed);
    rc |= get_qt(c, "lm_head.weight", s->vocab_size, hd, &m->lm_head);
    m->final_norm = get_vec(c, "model.norm.weight", hd);
    m->layers = (layer_w *)xcalloc((size_t)s->num_hidden_layers, sizeof(layer_w));
    for (int64_t li = 0; li < s->num_hidden_layers; li++)
        rc |= load_layer(c, s, li, li < s->first_k_dense_replace, &m->layers[li]);
    char nm[200];
    int64_t L = s->num_hidden_layers;
    snprintf(nm, sizeof nm, "model.layers.%lld.eh_proj.weight", (long long)L);
    if (s->mtp && find(c, nm)) {
        m->has_mtp = 1;
        rc |= get_qt(c, nm, hd, 2 * hd, &m->eh_proj);
        snprintf(nm, sizeof nm, "model.layers.%lld.enorm.weight", (long long)L); m->enorm = get_vec(c, nm, hd);
        snprintf(nm, sizeof nm, "model.layers.%lld.hnorm.weight", (long long)L); m->hnorm = get_vec(c, nm, hd);
        rc |= load_layer(c, s, L, 0, &m->mtp_layer);
        snprintf(nm, sizeof nm, "model.layers.%lld.shared_head.norm.weight", (long long)L); m->mtp_norm = get_vec(c, nm, hd);
        snprintf(nm, sizeof nm, "model.layers.%lld.shared_head.head.weight", (long long)L);
        rc |= get_qt(c, nm, s->vocab_size, hd, &m->mtp_head);
        if (!m->enorm || !m->hnorm || !m->mtp_norm) rc = -1;
    }
    if (rc || !m->final_norm) { uto_model_free(m); return NULL; }
    return m;
}

void uto_model_free(uto_model *m) {
    if (!m) return;
    if (m->layers) {
        for (int64_t li = 0; li < m->c.num_hidden_layers; li++) free(m->layers[li].experts);
        free(m->layers);
    }
    free(m->mtp_layer.experts);
    free(m);
}

/* ------------------------------------------------------------ KV cache -- */
typedef struct { float *latent, *k_rot; int64_t len, cap; } kv_cache;

static void kv_reserve(kv_cache *kv, int64_t total, int64_t L, int64_t P) {
    if (total <= kv->cap) return;
    int64_t nc = kv->cap ? kv->cap : 16;
    while (nc < total) nc *= 2;
    kv->latent = (float *)realloc(kv->latent, (size_t)(nc * L) * 4);
    kv->k_rot = (float *)realloc(kv->k_rot, (size_t)(nc * P) * 4);
    if (!kv->latent || !kv->k_rot) abort();
    kv->cap = nc;
}

/* mla_forward_cached (attention.rs:123-279); x [seq, hidden] is normed. */
static void mla_forward(const uto_spec *c, const layer_w *w, const float *x, int64_t seq,
                        kv_cache *kv, int path, float *out) {
    int64_t hd = c->hidden_size, h = c->num_attention_heads;
    int64_t nope = c->qk_nope_head_dim, rope = c->qk_rope_head_dim, vh = c->v_head_dim;
    int64_t Lr = c->kv_lora_rank, qh = nope + rope, kvh = nope + vh;
    float scale = 1.0f / sqrtf((float)qh); /* config.rs:142-144 */
    int64_t pos_base = kv->len, total = pos_base + seq;

    float *q = (float *)xcalloc((size_t)(seq * h * qh), 4);
    if (w->lora) {
        int64_t rank = w->q_a.out_dim;
        float *resid = (float *)xcalloc((size_t)rank, 4), *normed = (float *)xcalloc((size_t)rank, 4);
        for (int64_t s = 0; s < seq; s++) {
            qt_matmul(&w->q_a, x + s * hd, 1, resid);
            uto_rmsnorm(normed, resid, w->q_a_norm, rank, c->rms_norm_eps);
            qt_matmul(&w->q_b, normed, 1, q + s * h * qh);
        }
        free(resid); free(normed);
    } else {
        qt_matmul(&w->q_proj, x, seq, q);
    }
    for (int64_t s = 0; s < seq; s++)
        for (int64_t hh = 0; hh < h; hh++)
            uto_rope_interleave(q + s * h * qh + hh * qh + nope, pos_base + s, rope, c->rope_theta);

    kv_reserve(kv, total, Lr, rope);
    float *comp = (float *)xcalloc((size_t)(Lr + rope), 4);
    for (int64_t s = 0; s < seq; s++) {
        int64_t pos = pos_base + s;
        qt_matmul(&w->kv_a, x + s * hd, 1, comp);
        uto_rmsnorm(kv->latent + pos * Lr, comp, w->kv_a_norm, Lr, c->rms_norm_eps);
        float *kr = kv->k_rot + pos * rope;
        memcpy(kr, comp + Lr, (size_t)rope * 4);
        uto_rope_interleave(kr, pos, rope, c->rope_theta);
    }
    free(comp);
    kv->len = total;

    int absorbed = path == 1 ? 1 : (path == 2 ? 0 : seq <= 4);
    float *ctx = (float *)xcalloc((size_t)(seq * h * vh), 4);
    float *scores = (float *)xcalloc((size_t)total, 4);
    if (absorbed) {
        /* one task per (row, head), as the reference's rayon tasks
         * (attention.rs:202); each keeps its sequential order */
#pragma omp parallel for collapse(2) schedule(dynamic) if (seq * h * total >= (1 << 12))
        for (int64_t s = 0; s < seq; s++) {
            for (int64_t hh = 0; hh < h; hh++) {
                float *qabs = (float *)xcalloc((size_t)Lr, 4), *clat = (float *)xcalloc((size_t)Lr, 4);
                float *scores = (float *)xcalloc((size_t)total, 4);
                int64_t n_ctx = pos_base + s + 1;
                const float *qn = q + s * h * qh + hh * qh, *qr = qn + nope;
                int64_t rbase = hh * kvh;
                memset(qabs, 0, (size_t)Lr * 4);
                for (int64_t dd = 0; dd < nope; dd++)
                    uto_add_scaled_row(w->kv_b.fmt, w->kv_b.p, w->kv_b.s, w->kv_b.out_dim, Lr,
                                       rbase + dd, qn[dd], qabs);
                for (int64_t t = 0; t < n_ctx; t++) {
                    const float *lat = kv->latent + t * Lr, *kr = kv->k_rot + t * rope;
                    float a = 0.0f;
                    for (int64_t i = 0; i < Lr; i++) a += qabs[i] * lat[i];
                    for (int64_t i = 0; i < rope; i++) a += qr[i] * kr[i];
                    scores[t] = a * scale;
                }
                uto_softmax(scores, n_ctx);
                memset(clat, 0, (size_t)Lr * 4);
                for (int64_t t = 0; t < n_ctx; t++) {
                    const float *lat = kv->latent + t * Lr;
                    float a = scores[t];
                    for (int64_t i = 0; i < Lr; i++) clat[i] += a * lat[i];
                }
                uto_matvec_rows(w->kv_b.fmt, w->kv_b.p, w->kv_b.s, w->kv_b.out_dim, Lr,
                                rbase + nope, vh, clat, ctx + (s * h + hh) * vh);
                free(qabs); free(clat); free(scores);
            }
        }
    } else {
        float *kvr = (float *)xcalloc((size_t)(total * h * kvh), 4);
        qt_matmul(&w->kv_b, kv->latent, total, kvr);
        for (int64_t s = 0; s < seq; s++) {
            for (int64_t hh = 0; hh < h; hh++) {
                int64_t n_ctx = pos_base + s + 1;
                const float *qn = q + s * h * qh + hh * qh, *qr = qn + nope;
                for (int64_t t = 0; t < n_ctx; t++) {
                    const float *kn = kvr + t * h * kvh + hh * kvh, *kr = kv->k_rot + t * rope;
                    float a = 0.0f;
                    for (int64_t i = 0; i < nope; i++) a += qn[i] * kn[i];
                    for (int64_t i = 0; i < rope; i++) a += qr[i] * kr[i];
                    scores[t] = a * scale;
                }
                uto_softmax(scores, n_ctx);
                float *cx = ctx + (s * h + hh) * vh;
                for (int64_t i = 0; i < vh; i++) cx[i] = 0.0f;
                for (int64_t t = 0; t < n_ctx; t++) {
                    const float *vv = kvr + t * h * kvh + hh * kvh + nope;
                    float a = scores[t];
                    for (int64_t i = 0; i < vh; i++) cx[i] += a * vv[i];
                }
            }
        }
        free(kvr);
    }
    qt_matmul(&w->o_proj, ctx, seq, out);
    free(scores); free(ctx); free(q);
}

/* moe_forward (model.rs:195-286), accumulated into zeroed out. */
static void moe_forward(const uto_spec *c, const layer_w *w, const float *x, int64_t seq, float *out) {
    int64_t hd = c->hidden_size, inter = c->moe_intermediate_size, E = c->n_routed_experts;
    int64_t k = c->num_experts_per_tok;
    float *logits = (float *)xcalloc((size_t)E, 4);
    int64_t *ids = (int64_t *)xcalloc((size_t)k, 8);
    float *wts = (float *)xcalloc((size_t)k, 4);
    float *g = (float *)xcalloc((size_t)inter, 4), *u = (float *)xcalloc((size_t)inter, 4);
    float *d = (float *)xcalloc((size_t)hd, 4);
    for (int64_t s = 0; s < seq; s++) {
        const float *xs = x + s * hd;
        uto_matmul(UTO_F32, w->gate, NULL, E, hd, xs, 1, logits);
        uto_route(logits, w->bias, E, k, c->n_group, c->topk_group, c->norm_topk_prob,
                  c->routed_scaling_factor, ids, wts);
        float *os = out + s * hd;
        for (int64_t j = 0; j < k; j++) {
            const mlp_w *ex = &w->experts[ids[j]];
            qt_matmul(&ex->gate, xs, 1, g);
            qt_matmul(&ex->up, xs, 1, u);
            for (int64_t i = 0; i < inter; i++) g[i] = uto_silu(g[i]) * u[i];
            qt_matmul(&ex->down, g, 1, d);
            for (int64_t i = 0; i < hd; i++) os[i] += wts[j] * d[i];
        }
    }
    if (w->has_shared) {
        const mlp_w *sh = &w->shared;
        uto_mlp_forward_add(sh->gate.fmt, hd, sh->gate.out_dim, sh->gate.p, sh->gate.s, sh->up.p,
                            sh->up.s, sh->down.p, sh->down.s, x, seq, out);
    }
    free(logits); free(ids); free(wts); free(g); free(u); free(d);
}

/* run_layer (model.rs:127-183) / the per-layer body of prefill (:470-526). */
static void run_layer(const uto_spec *c, const layer_w *L, float *x, int64_t seq, kv_cache *kv, int path) {
    int64_t hd = c->hidden_size;
    float *normed = (float *)xcalloc((size_t)(seq * hd), 4);
    float *attn = (float *)xcalloc((size_t)(seq * hd), 4);
    for (int64_t s = 0; s < seq; s++) uto_rmsnorm(normed + s * hd, x + s * hd, L->input_norm, hd, c->rms_norm_eps);
    mla_forward(c, L, normed, seq, kv, path, attn);
    for (int64_t i = 0; i < seq * hd; i++) x[i] += attn[i];
    for (int64_t s = 0; s < seq; s++) uto_rmsnorm(normed + s * hd, x + s * hd, L->post_norm, hd, c->rms_norm_eps);
    if (L->dense) {
        const mlp_w *m = &L->mlp;
        uto_mlp_forward_add(m->gate.fmt, hd, m->gate.out_dim, m->gate.p, m->gate.s, m->up.p, m->up.s,
                            m->down.p, m->down.s, normed, seq, x);
    } else {
        float *moe = (float *)xcalloc((size_t)(seq * hd), 4);
        moe_forward(c, L, normed, seq, moe);
        for (int64_t i = 0; i < seq * hd; i++) x[i] += moe[i];
        free(moe);
    }
    free(normed); free(attn);
}

struct uto_session {
    uto_model *m;
    kv_cache *kv;
    int64_t pos;
    int path;
    int32_t *tokens;
    float *hidden;
    int64_t hcap;
};

uto_session *uto_session_new(uto_model *m, int path) {
    uto_session *s = (uto_session *)xcalloc(1, sizeof(uto_session));
    s->m = m;
    s->kv = (kv_cache *)xcalloc((size_t)m->c.num_hidden_layers, sizeof(kv_cache));
    s->path = path;
    return s;
}

void uto_session_free(uto_session *s) {
    if (!s) return;
    for (int64_t li = 0; li < s->m->c.num_hidden_layers; li++) { free(s->kv[li].latent); free(s->kv[li].k_rot); }
    free(s->kv); free(s->tokens); free(s->hidden); free(s);
}

static void embed_row(const uto_model *m, int64_t id, float *out) {
    /* model.rs:119-122 */
    memset(out, 0, (size_t)m->c.hidden_size * 4);
    uto_add_scaled_row(m->embed.fmt, m->embed.p, m->embed.s, m->embed.out_dim, m->embed.in_dim, id, 1.0f, out);
}

int uto_session_prefill(uto_session *s, const int32_t *ids, int64_t n, float *logits) {
    /* InferenceSession::prefill (model.rs:447-547) */
    const uto_model *m = s->m;
    const uto_spec *c = &m->c;
    int64_t hd = c->hidden_size, V = c->vocab_size;
    if (n <= 0) return -1;
    if (s->pos + n > c->max_position_embeddings) return -2;
    for (int64_t i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] >= V) return -3;
    float *x = (float *)xcalloc((size_t)(n * hd), 4);
    for (int64_t i = 0; i < n; i++) embed_row(m, ids[i], x + i * hd);
    for (int64_t li = 0; li < c->num_hidden_layers; li++)
        run_layer(c, &m->layers[li], x, n, &s->kv[li], s->path);
    s->pos += n;
    /* session.tokens always; session.hidden (the MTP head's input) with MTP */
    if (s->pos > s->hcap) {
        int64_t nc = s->hcap ? s->hcap : 64;
        while (nc < s->pos) nc *= 2;
        s->tokens = (int32_t *)realloc(s->tokens, (size_t)nc * 4);
        if (m->has_mtp) s->hidden = (float *)realloc(s->hidden, (size_t)(nc * hd) * 4);
        if (!s->tokens || (m->has_mtp && !s->hidden)) abort();
        s->hcap = nc;
    }
    memcpy(s->tokens + s->pos - n, ids, (size_t)n * 4);
    if (m->has_mtp) memcpy(s->hidden + (s->pos - n) * hd, x, (size_t)(n * hd) * 4);
    float *normed = (float *)xcalloc((size_t)hd, 4);
    for (int64_t i = 0; i < n; i++) {
        uto_rmsnorm(normed, x + i * hd, m->final_norm, hd, c->rms_norm_eps);
        if (logits) qt_matmul(&m->lm_head, normed, 1, logits + i * V);
    }
    free(normed); free(x);
    return 0;
}

void uto_session_truncate(uto_session *s, int64_t len) {
    /* model.rs:556-564, LayerKvCache::truncate (attention.rs:89-93) */
    for (int64_t li = 0; li < s->m->c.num_hidden_layers; li++)
        if (len < s->kv[li].len) s->kv[li].len = len;
    if (len < s->pos) s->pos = len;
}

int64_t uto_session_position(const uto_session *s) { return s->pos; }

/* ================================================== generation loops ==== */
/* The emit rule of undertow_core::generate (core/model.rs:139-166) and the
 * speculative loops (mtp.rs:194-257, 263-314): emit, report to on_token,
 * end after a stop token (emitted and counted), when on_token returns 0, or
 * at max_new tokens. */
typedef struct {
    const int32_t *stops;
    int64_t n_stops;
    uto_token_fn on_token;
    void *user;
    int32_t *out;
    int64_t max_new, produced;
} emit_state;

static int emit(emit_state *e, int32_t tok) {
    e->out[e->produced++] = tok;
    int keep = e->on_token ? e->on_token(e->user, tok) != 0 : 1;
    int stop = 0;
    for (int64_t i = 0; i < e->n_stops; i++)
        if (e->stops[i] == tok) stop = 1;
    return stop || !keep || e->produced >= e->max_new;
}

int64_t uto_generate_greedy(uto_model *m, const int32_t *prompt, int64_t n, int64_t max_new,
                            const int32_t *stops, int64_t n_stops, uto_token_fn on_token,
                            void *user, int32_t *out) {
    /* core/model.rs:139-166 with a greedy sampler (argmax). */
    int64_t V = m->c.vocab_size;
    uto_session *s = uto_session_new(m, 0);
    float *logits = (float *)xcalloc((size_t)(n * V), 4);
    int rc = uto_session_prefill(s, prompt, n, logits);
    if (rc) { free(logits); uto_session_free(s); return rc; }
    float *last = (float *)xcalloc((size_t)V, 4);
    memcpy(last, logits + (n - 1) * V, (size_t)V * 4);
    emit_state e = {stops, n_stops, on_token, user, out, max_new, 0};
    while (e.produced < max_new) {
        int32_t next = (int32_t)uto_argmax(last, V);
        if (emit(&e, next)) break;
        if (uto_session_prefill(s, &next, 1, last) == -2) break;
    }
    free(last); free(logits); uto_session_free(s);
    return e.produced;
}

int64_t uto_greedy_decode(uto_model *m, const int32_t *prompt, int64_t n, int64_t max_new, int32_t *out) {
    /* greedy_decode (core/model.rs:168-185) without stop ids. */
    return uto_generate_greedy(m, prompt, n, max_new, NULL, 0, NULL, NULL, out);
}

/* MtpState (mtp.rs:48-55): the MTP layer's own KV and the fed count. */
struct uto_mtp_state { kv_cache kv; int64_t fed; };

uto_mtp_state *uto_mtp_state_new(void) { return (uto_mtp_state *)xcalloc(1, sizeof(uto_mtp_state)); }

void uto_mtp_state_free(uto_mtp_state *st) {
    if (!st) return;
    free(st->kv.latent); free(st->kv.k_rot); free(st);
}

/* The MTP module over `rows` inputs: x_j = eh_proj(concat(enorm(embed(t_j)),
 * hnorm(h_j))), the MTP layer on its own KV, then the head over the last
 * row (mtp.rs:84-131).  last_out (may be NULL) gets the layer's output row
 * for the last input, before the head's norm. */
static void mtp_rows(uto_model *m, uto_mtp_state *st, const int32_t *t_next, const float *hidden,
                     int64_t rows, float *logits, float *last_out) {
    const uto_spec *c = &m->c;
    int64_t hd = c->hidden_size;
    float *xs = (float *)xcalloc((size_t)(rows * hd), 4);
    float *emb = (float *)xcalloc((size_t)hd, 4), *cat = (float *)xcalloc((size_t)(2 * hd), 4);
    for (int64_t j = 0; j < rows; j++) {
        embed_row(m, t_next[j], emb);
        uto_rmsnorm(cat, emb, m->enorm, hd, c->rms_norm_eps);
        uto_rmsnorm(cat + hd, hidden + j * hd, m->hnorm, hd, c->rms_norm_eps);
        qt_matmul(&m->eh_proj, cat, 1, xs + j * hd);
    }
    run_layer(c, &m->mtp_layer, xs, rows, &st->kv, 0);
    if (last_out) memcpy(last_out, xs + (rows - 1) * hd, (size_t)hd * 4);
    float *normed = (float *)xcalloc((size_t)hd, 4);
    uto_rmsnorm(normed, xs + (rows - 1) * hd, m->mtp_norm, hd, c->rms_norm_eps);
    qt_matmul(&m->mtp_head, normed, 1, logits);
    free(normed); free(emb); free(cat); free(xs);
}

int uto_draft_logits(uto_model *m, uto_session *sess, uto_mtp_state *st, int32_t next_token,
                     float *logits, float *last_out) {
    /* draft_logits (mtp.rs:74-133): pending positions fed..pos-1, t_next =
     * the following consumed token, next_token for the last. */
    if (!m->has_mtp) return -4;
    int64_t pos = sess->pos, pending = pos - st->fed;
    if (pending <= 0) return -5;
    int32_t *t_next = (int32_t *)xcalloc((size_t)pending, 4);
    for (int64_t j = 0, i = st->fed; i < pos; i++, j++)
        t_next[j] = i + 1 < pos ? sess->tokens[i + 1] : next_token;
    mtp_rows(m, st, t_next, sess->hidden + st->fed * m->c.hidden_size, pending, logits, last_out);
    st->fed = pos;
    free(t_next);
    return 0;
}

int64_t uto_speculative_loop(uto_model *m, const int32_t *prompt, int64_t n, int64_t max_new,
                             int32_t depth, const int32_t *stops, int64_t n_stops,
                             uto_token_fn on_token, void *user, uto_draft_fn draft_fn,
                             void *draft_user, int32_t *out, int64_t *drafted, int64_t *accepted) {
    /* speculative_loop (mtp.rs:263-314); the greedy path of
     * speculative_loop_with_sampler (mtp.rs:194-257) makes the same
     * decisions (one-hot p and q).  depth 1 is the reference.  depth 2..3
     * (an extension): the native head chains the MTP layer on its own output
     * row for the last fed position with the previous draft's embedding
     * (rows never kept: the MTP KV returns to the fed length), the verify
     * prefill takes [next, d1..dk] and the longest prefix of drafts equal to
     * the verify argmax rows is accepted. */
    if (drafted) *drafted = 0;
    if (accepted) *accepted = 0;
    if (depth < 1 || depth > 3) return -1;
    if (!draft_fn && !m->has_mtp) return -4;
    int64_t V = m->c.vocab_size, hd = m->c.hidden_size;
    uto_session *s = uto_session_new(m, 0);
    uto_mtp_state *st = uto_mtp_state_new();
    float *logits = (float *)xcalloc((size_t)(n * V), 4);
    int rc = uto_session_prefill(s, prompt, n, logits);
    if (rc) { free(logits); uto_mtp_state_free(st); uto_session_free(s); return rc; }
    int32_t next = (int32_t)uto_argmax(logits + (n - 1) * V, V);
    float *dl = (float *)xcalloc((size_t)V, 4), *ver = (float *)xcalloc((size_t)((depth + 1) * V), 4);
    float *row = (float *)xcalloc((size_t)hd, 4), *row2 = (float *)xcalloc((size_t)hd, 4);
    int32_t d[3], vid[4];
    int64_t nd = 0, na = 0;
    emit_state e = {stops, n_stops, on_token, user, out, max_new, 0};
    int64_t result = 0;
    if (max_new == 0) goto done;
    for (;;) {
        if (emit(&e, next)) break;
        if (draft_fn) {
            int32_t r = draft_fn(draft_user, s->tokens, s->pos, next, depth, d);
            if (r < 0) { result = r; goto done; }
            for (int i = 0; i < depth; i++)
                if (d[i] < 0 || d[i] >= V) { result = -3; goto done; }
        } else {
            uto_draft_logits(m, s, st, next, dl, row);
            d[0] = (int32_t)uto_argmax(dl, V);
            int64_t kv_len = st->kv.len;
            for (int j = 1; j < depth; j++) {
                mtp_rows(m, st, &d[j - 1], row, 1, dl, row2);
                memcpy(row, row2, (size_t)hd * 4);
                d[j] = (int32_t)uto_argmax(dl, V);
            }
            st->kv.len = kv_len;
        }
        nd += depth;
        int64_t pos_before = s->pos;
        vid[0] = next;
        for (int i = 0; i < depth; i++) vid[i + 1] = d[i];
        if (uto_session_prefill(s, vid, depth + 1, ver) == -2) break;
        int64_t a = 0;
        int end = 0;
        while (a < depth && (int32_t)uto_argmax(ver + a * V, V) == d[a]) {
            a++;
            na++;
            if (emit(&e, d[a - 1])) { end = 1; break; }
        }
        if (end) break;
        next = (int32_t)uto_argmax(ver + a * V, V);
        if (a < depth) uto_session_truncate(s, pos_before + 1 + a);
    }
    result = e.produced;
done:
    if (drafted) *drafted = nd;
    if (accepted) *accepted = na;
    free(dl); free(ver); free(logits); free(row); free(row2);
    uto_mtp_state_free(st);
    uto_session_free(s);
    return result;
}

int64_t uto_generate_mtp(uto_model *m, const int32_t *prompt, int64_t n, int64_t max_new, int32_t *out,
                         int64_t *drafted, int64_t *accepted) {
    /* generate_greedy_mtp (mtp.rs:176-191) without stop ids: depth 1. */
    return uto_speculative_loop(m, prompt, n, max_new, 1, NULL, 0, NULL, NULL, NULL, NULL, out,
                                drafted, accepted);
}
