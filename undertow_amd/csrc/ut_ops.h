// ut_ops.h -- the small per-layer kernels of the decode step.
#pragma once

#include "ut_internal.h"

namespace ut {

// Code i of a quantized row as a float (f32 rows: the value).
__device__ __forceinline__ float code_at(int32_t fmt, const uint8_t *row, int64_t i) {
    if (fmt == UT_FMT_F32) return ((const float *)row)[i];
    if (fmt == UT_FMT_INT8) return (float)(int8_t)row[i];
    uint8_t b = row[i >> 1];
    int nib = (i & 1) ? (b >> 4) : (b & 0xF);
    return (float)((nib ^ 8) - 8);
}

// One cache append (attention.rs:168-186): latent[pos] = rmsnorm(c[:L], w),
// krot[pos] = rope_interleave(c[L:L+P], pos), by the whole workgroup (up to
// 1024 threads; red: one double per wave).
// kc != nullptr: the cache is kept in the split bf16 form of the MFMA
// attention kernel (per position: hi parts of [latent | k_rot], then lo).
// c may point to global or shared memory.  red: 4 doubles of shared memory.
__device__ __forceinline__ void kv_store(float *__restrict__ plain, int64_t pi,
                                         __bf16 *__restrict__ kc, int64_t ki, int64_t D, float v) {
    if (kc) {
        const __bf16 h = (__bf16)v;
        kc[ki] = h;
        kc[ki + D] = (__bf16)__fsub_rn(v, (float)h);
    } else {
        plain[pi] = v;
    }
}

__device__ __forceinline__ void kv_append_row(const float *c, int64_t L, int64_t P,
                                              const float *__restrict__ w, float eps,
                                              float *__restrict__ latent, float *__restrict__ krot,
                                              __bf16 *__restrict__ kc, int64_t pos,
                                              const float2 *__restrict__ table, double *red) {
    const int nt = blockDim.x, nw = nt >> 6;
    double acc = 0.0;
    for (int64_t i = threadIdx.x; i < L; i += nt) {
        const double v = (double)c[i];
        acc += v * v;
    }
    for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    // waves summed pairwise in a fixed tree ((0+1)+(2+3)) + ... for 4 waves
    double ms = 0.0;
    for (int q = 0; q < nw; q += 4) {
        double t = red[q];
        if (q + 1 < nw) t += red[q + 1];
        double t2 = q + 2 < nw ? red[q + 2] : 0.0;
        if (q + 3 < nw) t2 += red[q + 3];
        ms += t + t2;
    }
    ms /= (double)L;
    const float r = 1.0f / sqrtf(__fadd_rn((float)ms, eps));
    const int64_t D = L + P, kb = pos * 2 * D;
    for (int64_t i = threadIdx.x; i < L; i += nt)
        kv_store(latent, pos * L + i, kc, kb + i, D, __fmul_rn(__fmul_rn(c[i], r), w[i]));
    const int64_t half = P / 2;
    for (int64_t jj = threadIdx.x; jj < P; jj += nt) {
        const int64_t j = jj < half ? jj : jj - half;
        const float a = c[L + 2 * j], b = c[L + 2 * j + 1];
        const float2 cs = table[pos * half + j];
        kv_store(krot, pos * P + jj, kc, kb + L + jj, D,
                 jj < half ? __fsub_rn(__fmul_rn(a, cs.x), __fmul_rn(b, cs.y))
                           : __fadd_rn(__fmul_rn(b, cs.x), __fmul_rn(a, cs.y)));
    }
}

// Embedding rows (model.rs:119-122): out[s] = 0 + (1*scale[id])*q[id] (f32
// tables copied).  ids: device int32 [rows].
int32_t launch_embed(ut_ctx *ctx, const ut_qtensor *emb, const int32_t *ids, int64_t rows,
                     float *out, int64_t ldo);
// rmsnorm (undertow-quant/src/lib.rs:91-100) per row: the mean of squares in
// f64, r = 1/sqrt((float)ms + eps), out = (x*r)*w.
int32_t launch_rmsnorm(ut_ctx *ctx, const float *x, int64_t ldx, const float *w, int64_t n,
                       float eps, int64_t rows, float *out, int64_t ldo);
// y += x (f32 adds), n elements.
int32_t launch_add(ut_ctx *ctx, float *y, const float *x, int64_t n);
// bf16 -> f32 (exact widening), n elements.
int32_t launch_bf16_to_f32(ut_ctx *ctx, const uint16_t *x, int64_t n, float *y);
// dst rows [pos, pos + rows) (stride ld) <- src [rows][H]; pos follows the
// context's captured-step position when one is set.
int32_t launch_copy_rows_at(ut_ctx *ctx, float *dst, int64_t ld, int64_t pos, const float *src,
                            int64_t rows, int64_t H);
// dst [rows][H] <- src rows [pos, pos + rows) (stride ld); pos as above.
int32_t launch_copy_rows_from(ut_ctx *ctx, float *dst, const float *src, int64_t ld, int64_t pos,
                              int64_t rows, int64_t H);
// The MTP feed's ids after a verify that accepted a drafts: vids[1..a], am[a].
int32_t launch_feed_ids(ut_ctx *ctx, int32_t *dst, const int32_t *vids, const int32_t *am, int a);
// *p = v, and *p += n (a captured step's position word).
int32_t launch_pos_set(ut_ctx *ctx, int64_t *p, int64_t v);
int32_t launch_pos_add(ut_ctx *ctx, int64_t *p, int64_t n);
// Absorbed query (attention.rs:204-213): for each (s, h)
//   qabs[s,h,:] = sum_d (q[s,h,d]*scale[h*kvh+d]) * W[h*kvh+d, :]  (d < nope,
//   adds in d order) and q_rope[s,h,:] = rope_interleave(q[s,h,nope:], pos_base+s).
int32_t launch_absorb_q(ut_ctx *ctx, const ut_qtensor *kv_b, const float *q, int64_t rows,
                        int64_t heads, int64_t nope, int64_t rope, int64_t vh, float *qabs,
                        float *qrope, int64_t pos_base, const float2 *table);
// Cache append (attention.rs:168-186) for rows at positions pos_base..:
// latent = rmsnorm(comp[:L], w), krot = rope_interleave(comp[L:L+P], pos),
// stored as f32 (latent, krot) or, with kc, in the MFMA attention's split
// bf16 form (per position: hi parts of [latent | krot], then lo parts).
int32_t launch_kv_append(ut_ctx *ctx, const float *comp, int64_t rows, int64_t L, int64_t P,
                         const float *w, float eps, float *latent, float *krot, __bf16 *kc,
                         int64_t pos_base, const float2 *table);
// Absorbed value (attention.rs:235, QTensor::matvec_rows): for each (s, h)
//   ctx[s, h*vh + j] = (sum_i clat[s,h,i] * W[h*kvh+nope+j, i]) * scale.
// vmax (optional, absorb_v_max_ok weights): partial maxima of |ctx| per row,
// [rows][absorb_v_parts(heads, vh)] float bits, for the o_proj GEMV's
// digitising.
bool absorb_v_max_ok(const ut_qtensor *kv_b);
int64_t absorb_v_parts(int64_t heads, int64_t vh);
int32_t launch_absorb_v(ut_ctx *ctx, const ut_qtensor *kv_b, const float *clat, int64_t rows,
                        int64_t heads, int64_t nope, int64_t vh, float *out,
                        uint32_t *vmax = nullptr);

}  // namespace ut
