/*
 * cpu_baseline.c -- the reference's *dispatched* CPU path, restated in C, for
 * timing only.  TEST/BENCH INFRASTRUCTURE: bench.py's cpu_baseline leg is the
 * only caller.  Never linked into the product library.
 *
 * What it restates:
 *   - avx512::dot_i4 / dot_i8 (undertow-quant/src/avx512.rs:62-83,118-156):
 *     two 16-lane f32 accumulators over 32-element chunks, nibble interleave
 *     plus shift-12 sign extension, reduce, scalar tail;
 *   - avx2::dot_i4 / dot_i8 (undertow-quant/src/avx2.rs:53-110) as the
 *     fallback when AVX-512 is absent; scalar kernels otherwise;
 *   - the rayon fan-out of QTensor::matmul (qtensor.rs:281-319) and of
 *     moe_forward's par_iter over unique experts (model.rs:236-261), mapped
 *     onto one OpenMP parallel-for over (expert, output-row block) tasks;
 *   - the absorbed MLA loops, one task per (row, head) (attention.rs:202-236).
 * Results match the scalar oracle up to f32 lane reassociation (the
 * reference's own SIMD-vs-scalar bound is 1e-4 relative, avx512.rs:335-366).
 */
#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { F_INT8 = 1, F_INT4 = 2 };

static int8_t unpack_i4(const uint8_t *row, int64_t i) {
    uint8_t b = row[i / 2];
    uint8_t nib = (i % 2 == 0) ? (uint8_t)(b & 0x0F) : (uint8_t)(b >> 4);
    return (int8_t)((int8_t)(nib << 4) >> 4);
}

/* ------------------------------------------------------------ AVX-512 --- */
__attribute__((target("avx512f,avx512bw,avx512dq,avx512vl")))
static float dot_i4_avx512(const float *x, const uint8_t *packed, int64_t n) {
    __m512 acc0 = _mm512_setzero_ps(), acc1 = _mm512_setzero_ps();
    const __m128i low = _mm_set1_epi8(0x0F);
    int64_t chunks = n / 32;
    for (int64_t c = 0; c < chunks; c++) {
        __m128i bytes = _mm_loadu_si128((const __m128i *)(packed + c * 16));
        __m128i even = _mm_and_si128(bytes, low);
        __m128i odd = _mm_and_si128(_mm_srli_epi16(bytes, 4), low);
        __m128i il = _mm_unpacklo_epi8(even, odd), ih = _mm_unpackhi_epi8(even, odd);
        __m128i sl0 = _mm_srai_epi16(_mm_slli_epi16(_mm_cvtepi8_epi16(il), 12), 12);
        __m128i sl1 = _mm_srai_epi16(_mm_slli_epi16(_mm_cvtepi8_epi16(_mm_srli_si128(il, 8)), 12), 12);
        __m128i sh0 = _mm_srai_epi16(_mm_slli_epi16(_mm_cvtepi8_epi16(ih), 12), 12);
        __m128i sh1 = _mm_srai_epi16(_mm_slli_epi16(_mm_cvtepi8_epi16(_mm_srli_si128(ih, 8)), 12), 12);
        __m512 f0 = _mm512_cvtepi32_ps(_mm512_cvtepi16_epi32(_mm256_set_m128i(sl1, sl0)));
        __m512 f1 = _mm512_cvtepi32_ps(_mm512_cvtepi16_epi32(_mm256_set_m128i(sh1, sh0)));
        int64_t i = c * 32;
        acc0 = _mm512_fmadd_ps(_mm512_loadu_ps(x + i), f0, acc0);
        acc1 = _mm512_fmadd_ps(_mm512_loadu_ps(x + i + 16), f1, acc1);
    }
    float acc = _mm512_reduce_add_ps(_mm512_add_ps(acc0, acc1));
    for (int64_t i = chunks * 32; i < n; i++) acc += x[i] * (float)unpack_i4(packed, i);
    return acc;
}

__attribute__((target("avx512f,avx512bw,avx512dq,avx512vl")))
static float dot_i8_avx512(const float *x, const int8_t *q, int64_t n) {
    __m512 acc0 = _mm512_setzero_ps(), acc1 = _mm512_setzero_ps();
    int64_t chunks = n / 32;
    for (int64_t c = 0; c < chunks; c++) {
        int64_t i = c * 32;
        __m256i qv = _mm256_loadu_si256((const __m256i *)(q + i));
        __m512 f0 = _mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(_mm256_castsi256_si128(qv)));
        __m512 f1 = _mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(_mm256_extracti128_si256(qv, 1)));
        acc0 = _mm512_fmadd_ps(_mm512_loadu_ps(x + i), f0, acc0);
        acc1 = _mm512_fmadd_ps(_mm512_loadu_ps(x + i + 16), f1, acc1);
    }
    float acc = _mm512_reduce_add_ps(_mm512_add_ps(acc0, acc1));
    for (int64_t i = chunks * 32; i < n; i++) acc += x[i] * (float)q[i];
    return acc;
}

/* --------------------------------------------------------------- AVX2 --- */
__attribute__((target("avx2,fma")))
static float hsum256(__m256 v) {
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 1));
    return _mm_cvtss_f32(s);
}

__attribute__((target("avx2,fma")))
static float dot_i4_avx2(const float *x, const uint8_t *packed, int64_t n) {
    __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
    const __m128i low = _mm_set1_epi8(0x0F);
    int64_t chunks = n / 16;
    for (int64_t c = 0; c < chunks; c++) {
        __m128i bytes = _mm_loadl_epi64((const __m128i *)(packed + c * 8));
        __m128i even = _mm_and_si128(bytes, low);
        __m128i odd = _mm_and_si128(_mm_srli_epi16(bytes, 4), low);
        __m128i inter = _mm_unpacklo_epi8(even, odd);
        __m128i s0 = _mm_srai_epi16(_mm_slli_epi16(_mm_cvtepi8_epi16(inter), 12), 12);
        __m128i s1 = _mm_srai_epi16(_mm_slli_epi16(_mm_cvtepi8_epi16(_mm_srli_si128(inter, 8)), 12), 12);
        __m256 f0 = _mm256_cvtepi32_ps(_mm256_cvtepi16_epi32(s0));
        __m256 f1 = _mm256_cvtepi32_ps(_mm256_cvtepi16_epi32(s1));
        int64_t i = c * 16;
        acc0 = _mm256_fmadd_ps(_mm256_loadu_ps(x + i), f0, acc0);
        acc1 = _mm256_fmadd_ps(_mm256_loadu_ps(x + i + 8), f1, acc1);
    }
    float acc = hsum256(acc0) + hsum256(acc1);
    for (int64_t i = chunks * 16; i < n; i++) acc += x[i] * (float)unpack_i4(packed, i);
    return acc;
}

__attribute__((target("avx2,fma")))
static float dot_i8_avx2(const float *x, const int8_t *q, int64_t n) {
    __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
    int64_t chunks = n / 16;
    for (int64_t c = 0; c < chunks; c++) {
        int64_t i = c * 16;
        __m128i qv = _mm_loadu_si128((const __m128i *)(q + i));
        __m256 f0 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(qv));
        __m256 f1 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(qv, 8)));
        acc0 = _mm256_fmadd_ps(_mm256_loadu_ps(x + i), f0, acc0);
        acc1 = _mm256_fmadd_ps(_mm256_loadu_ps(x + i + 8), f1, acc1);
    }
    float acc = hsum256(acc0) + hsum256(acc1);
    for (int64_t i = chunks * 16; i < n; i++) acc += x[i] * (float)q[i];
    return acc;
}

/* ------------------------------------------------------------- scalar --- */
static float dot_i4_scalar(const float *x, const uint8_t *packed, int64_t n) {
    float acc = 0.0f;
    for (int64_t i = 0; i < n; i++) acc += x[i] * (float)unpack_i4(packed, i);
    return acc;
}
static float dot_i8_scalar(const float *x, const int8_t *q, int64_t n) {
    float acc = 0.0f;
    for (int64_t i = 0; i < n; i++) acc += x[i] * (float)q[i];
    return acc;
}

static int g_isa = -1; /* 2 avx512, 1 avx2, 0 scalar */

int ucb_isa(void) {
    if (g_isa < 0) {
        __builtin_cpu_init();
        if (__builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
            __builtin_cpu_supports("avx512dq") && __builtin_cpu_supports("avx512vl"))
            g_isa = 2;
        else if (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma"))
            g_isa = 1;
        else
            g_isa = 0;
    }
    return g_isa;
}

/* Force an ISA (tests); -1 restores auto-detection. */
void ucb_set_isa(int isa) { g_isa = isa; if (isa < 0) (void)ucb_isa(); }

static float dot(int fmt, const float *x, const void *row, int64_t n) {
    int isa = ucb_isa();
    if (fmt == F_INT4) {
        if (isa == 2) return dot_i4_avx512(x, (const uint8_t *)row, n);
        if (isa == 1) return dot_i4_avx2(x, (const uint8_t *)row, n);
        return dot_i4_scalar(x, (const uint8_t *)row, n);
    }
    if (isa == 2) return dot_i8_avx512(x, (const int8_t *)row, n);
    if (isa == 1) return dot_i8_avx2(x, (const int8_t *)row, n);
    return dot_i8_scalar(x, (const int8_t *)row, n);
}

static int64_t row_bytes(int fmt, int64_t in_dim) { return fmt == F_INT4 ? (in_dim + 1) / 2 : in_dim; }

/* QTensor::matmul with the rayon split, threads = nthreads. */
void ucb_matmul(int fmt, const void *payload, const float *scales, int64_t out_dim, int64_t in_dim,
                const float *x, int64_t seq, float *out, int nthreads) {
    int64_t rb = row_bytes(fmt, in_dim);
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 16) collapse(2)
    for (int64_t s = 0; s < seq; s++)
        for (int64_t o = 0; o < out_dim; o++)
            out[s * out_dim + o] =
                dot(fmt, x + s * in_dim, (const uint8_t *)payload + o * rb, in_dim) * scales[o];
}

static float silu(float v) { return v / (1.0f + expf(-v)); }

/* moe_forward's expert block (model.rs:219-281) over host cores:
 * rows grouped by expert in first-appearance order, gate/up per (expert,
 * row-block) task, SiLU*mul, down per task, then the choice-order combine. */
void ucb_moe_experts(int fmt, int64_t hidden, int64_t inter, const uint8_t *gate_payload,
                     const float *gate_scales, const uint8_t *up_payload, const float *up_scales,
                     const uint8_t *down_payload, const float *down_scales, int64_t M,
                     int64_t top_k, const int64_t *ids, const float *weights, const float *x,
                     float *out, int nthreads) {
    int64_t gbytes = row_bytes(fmt, hidden) * inter, dbytes = row_bytes(fmt, inter) * hidden;
    int64_t grb = row_bytes(fmt, hidden), drb = row_bytes(fmt, inter);
    int64_t nslot = M * top_k;
    /* unique experts in first-appearance order; slot -> unique index */
    int64_t *uniq = (int64_t *)calloc((size_t)nslot, 8), *slot_u = (int64_t *)calloc((size_t)nslot, 8);
    int64_t nu = 0;
    for (int64_t q = 0; q < nslot; q++) {
        int64_t e = ids[q], u = -1;
        for (int64_t j = 0; j < nu; j++) if (uniq[j] == e) { u = j; break; }
        if (u < 0) { u = nu; uniq[nu++] = e; }
        slot_u[q] = u;
    }
    float *g = (float *)calloc((size_t)(nslot * inter), 4), *up = (float *)calloc((size_t)(nslot * inter), 4);
    float *d = (float *)calloc((size_t)(nslot * hidden), 4);
    if (nthreads > 0) omp_set_num_threads(nthreads);
    const int64_t BLK = 64;
    int64_t gblocks = (inter + BLK - 1) / BLK, dblocks = (hidden + BLK - 1) / BLK;
#pragma omp parallel
    {
#pragma omp for schedule(dynamic, 1)
        for (int64_t t = 0; t < nu * gblocks; t++) {
            int64_t u = t / gblocks, o0 = (t % gblocks) * BLK, o1 = o0 + BLK < inter ? o0 + BLK : inter;
            int64_t e = uniq[u];
            const uint8_t *gp = gate_payload + e * gbytes, *upp = up_payload + e * gbytes;
            for (int64_t q = 0; q < nslot; q++) {
                if (slot_u[q] != u) continue;
                const float *xs = x + (q / top_k) * hidden;
                for (int64_t o = o0; o < o1; o++) {
                    float gv = dot(fmt, xs, gp + o * grb, hidden) * gate_scales[e * inter + o];
                    float uv = dot(fmt, xs, upp + o * grb, hidden) * up_scales[e * inter + o];
                    g[q * inter + o] = gv;
                    up[q * inter + o] = uv;
                }
            }
        }
#pragma omp for schedule(static)
        for (int64_t i = 0; i < nslot * inter; i++) g[i] = silu(g[i]) * up[i];
#pragma omp for schedule(dynamic, 1)
        for (int64_t t = 0; t < nu * dblocks; t++) {
            int64_t u = t / dblocks, o0 = (t % dblocks) * BLK, o1 = o0 + BLK < hidden ? o0 + BLK : hidden;
            int64_t e = uniq[u];
            const uint8_t *dp = down_payload + e * dbytes;
            for (int64_t q = 0; q < nslot; q++) {
                if (slot_u[q] != u) continue;
                for (int64_t o = o0; o < o1; o++)
                    d[q * hidden + o] = dot(fmt, g + q * inter, dp + o * drb, inter) * down_scales[e * hidden + o];
            }
        }
    }
    memset(out, 0, (size_t)(M * hidden) * 4);
    for (int64_t s = 0; s < M; s++)
        for (int64_t c = 0; c < top_k; c++) {
            int64_t q = s * top_k + c;
            float w = weights[q];
            for (int64_t i = 0; i < hidden; i++) out[s * hidden + i] += w * d[q * hidden + i];
        }
    free(g); free(up); free(d); free(uniq); free(slot_u);
}

/* Absorbed MLA score/softmax/context loops, one task per (row, head)
 * (attention.rs:202-234). */
void ucb_mla_attend(const float *qabs, const float *q_rope, const float *latent, const float *krot,
                    int64_t R, int64_t H, int64_t L, int64_t P, int64_t pos_base, float scale,
                    float *clat, int nthreads) {
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
    {
        float *scores = (float *)malloc((size_t)(pos_base + R) * 4);
#pragma omp for schedule(dynamic, 1)
        for (int64_t k = 0; k < R * H; k++) {
            int64_t s = k / H, n_ctx = pos_base + s + 1;
            const float *qa = qabs + k * L, *qr = q_rope + k * P;
            float m = -INFINITY;
            for (int64_t t = 0; t < n_ctx; t++) {
                const float *lat = latent + t * L, *kr = krot + t * P;
                float a = 0.0f;
                for (int64_t i = 0; i < L; i++) a += qa[i] * lat[i];
                for (int64_t i = 0; i < P; i++) a += qr[i] * kr[i];
                scores[t] = a * scale;
                m = fmaxf(m, scores[t]);
            }
            float sum = 0.0f;
            for (int64_t t = 0; t < n_ctx; t++) { scores[t] = expf(scores[t] - m); sum += scores[t]; }
            for (int64_t t = 0; t < n_ctx; t++) scores[t] /= sum;
            float *cl = clat + k * L;
            for (int64_t i = 0; i < L; i++) cl[i] = 0.0f;
            for (int64_t t = 0; t < n_ctx; t++) {
                const float *lat = latent + t * L;
                float a = scores[t];
                for (int64_t i = 0; i < L; i++) cl[i] += a * lat[i];
            }
        }
        free(scores);
    }
}

int ucb_max_threads(void) { return omp_get_max_threads(); }
