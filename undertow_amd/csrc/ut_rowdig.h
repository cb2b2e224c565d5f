// ut_rowdig.h -- the row digitiser's shared pieces: rms-normalise a row held
// in registers (optionally), find its exponent and write its digit forms.
// Used by the digitiser launches and by kernels that finish a row and
// digitise it in the same launch.
#pragma once

#include "ut_gemv_core.h"
#include "ut_moe.h"

namespace ut {

// One activation row per workgroup.  x~ = rint(x * 2^(22-E)) with
// max|x| < 2^E (frexp), so |x~| <= 2^22 and six balanced base-16 digits
// (or three base-256 digits) represent it exactly.  With norm_w set, the
// row is first rms-normalised exactly as undertow-quant/src/lib.rs:91-100
// (mean of squares in f64, r = 1/sqrt((float)ms + eps), v = (x*r)*w) and the
// normalised row is what gets digitised (and optionally written out as f32).
struct RowDigArgs {
    const float *x;
    int64_t ldx, K;
    const float *norm_w;
    float eps;
    float *out;
    int64_t ldo;
    const uint32_t *rowmax;  // optional [rows][nparts] max|x| bits
    int32_t nparts;
    const int32_t *slot_count;
    int rows_per_slot;
    int32_t *exps;
    uint32_t *dig4, *dig8;
    int32_t *xt;
    // optional slot plan built by the launch's last workgroup
    const int32_t *plan_ids;
    int plan_M, plan_k, plan_E;
    const void *const *tbl;  // [6][E] expert pointer table
    MoePlan plan;
    int32_t *err_flag;
    // rowdig_body<GPT, true>: the incoming (un-normalised) row is stored
    // here (row stride ldr) after the reductions
    float *raw;
    int64_t ldr;
    // and, when set, also at row pos2 + m of raw2 (stride ldr2)
    float *raw2;
    int64_t ldr2;
    PosRef pos2;
};

template <typename T, typename Op>
__device__ __forceinline__ T wide_reduce(T v, Op op, T *red /* [16] */) {
    v = wave_reduce_dpp(v, op);
    const int nw = (blockDim.x + 63) >> 6;
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    // LDS-only barriers: the fence of __syncthreads would also wait for the
    // caller's outstanding global stores
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    T r = red[0];
    for (int w = 1; w < nw; w++) r = op(r, red[w]);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    return r;
}

// The part of the row digitiser after the row is in registers: thread tid
// owns the 8-column groups tid + g*blockDim.x (v zero past K), wv the norm
// weights of the same columns (read when a.norm_w is set).  RAW: also store
// the incoming row to a.raw -- after the reductions, so that their barriers
// do not wait for the stores (a producer that finishes the row hands it
// over here instead of storing it first).
template <int GPT, bool RAW = false>
__device__ __forceinline__ void rowdig_body(const RowDigArgs &a, int64_t m, float (&v)[GPT][8],
                                            const float (&wv)[GPT][8], double *redd,
                                            uint32_t *redu) {
    const int tid = threadIdx.x, nt = blockDim.x;
    const int64_t K = a.K, NG = (K + 7) / 8;
    float rv[RAW ? GPT : 1][8];
    if constexpr (RAW)
#pragma unroll
        for (int g = 0; g < GPT; g++)
#pragma unroll
            for (int j = 0; j < 8; j++) rv[g][j] = v[g][j];
    if (a.norm_w) {
        double acc = 0.0;
#pragma unroll
        for (int g = 0; g < GPT; g++)
#pragma unroll
            for (int j = 0; j < 8; j++) acc += (double)v[g][j] * (double)v[g][j];
        acc = wide_reduce(acc, [](double p, double q) { return p + q; }, redd);
        const float r = 1.0f / sqrtf(__fadd_rn((float)(acc / (double)K), a.eps));
#pragma unroll
        for (int g = 0; g < GPT; g++)
#pragma unroll
            for (int j = 0; j < 8; j++) v[g][j] = __fmul_rn(__fmul_rn(v[g][j], r), wv[g][j]);
    }
    uint32_t mx = 0;
#pragma unroll
    for (int g = 0; g < GPT; g++) {
        const int64_t c = tid + (int64_t)g * nt;
        if (c >= NG) continue;
#pragma unroll
        for (int j = 0; j < 8; j++) mx = max(mx, __float_as_uint(fabsf(v[g][j])));
    }
    if (a.rowmax) {
        mx = 0;
        for (int i = tid; i < a.nparts; i += nt) mx = max(mx, a.rowmax[m * a.nparts + i]);
    }
    mx = wide_reduce(mx, [](uint32_t p, uint32_t q) { return p > q ? p : q; }, redu);
    // every store comes after the last barrier, so no barrier waits for them
    if constexpr (RAW) {
        float *r2 = a.raw2 ? a.raw2 + (a.pos2.get() + m) * a.ldr2 : nullptr;
#pragma unroll
        for (int g = 0; g < GPT; g++) {
            const int64_t c = tid + (int64_t)g * nt;
            if (8 * c + 8 > K) continue;  // callers with RAW take whole groups
            float *o = a.raw + m * a.ldr + 8 * c;
            *(float4 *)o = make_float4(rv[g][0], rv[g][1], rv[g][2], rv[g][3]);
            *(float4 *)(o + 4) = make_float4(rv[g][4], rv[g][5], rv[g][6], rv[g][7]);
            if (r2) {
                *(float4 *)(r2 + 8 * c) = make_float4(rv[g][0], rv[g][1], rv[g][2], rv[g][3]);
                *(float4 *)(r2 + 8 * c + 4) = make_float4(rv[g][4], rv[g][5], rv[g][6], rv[g][7]);
            }
        }
    }
    if (a.out) {
        // whole 8-column groups of a 16-byte aligned row: two 16-byte stores
        const bool ovec = ((uintptr_t)(a.out + m * a.ldo) & 15) == 0;
#pragma unroll
        for (int g = 0; g < GPT; g++) {
            const int64_t c = tid + (int64_t)g * nt;
            if (c >= NG) continue;
            float *o = a.out + m * a.ldo + 8 * c;
            if (ovec && 8 * c + 8 <= K) {
                *(float4 *)o = make_float4(v[g][0], v[g][1], v[g][2], v[g][3]);
                *(float4 *)(o + 4) = make_float4(v[g][4], v[g][5], v[g][6], v[g][7]);
                continue;
            }
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (8 * c + j < K) o[j] = v[g][j];
        }
    }
    // non-finite rows (|x| bits >= +inf) produce NaN outputs downstream
    const bool bad = mx >= 0x7f800000u;
    int E = 0;
    if (!bad && mx != 0) (void)frexpf(__uint_as_float(mx), &E);
    const int sh = bad ? INT32_MIN : 22 - E;
    if (tid == 0) a.exps[m] = bad ? INT32_MIN : E - 22;
    const int64_t K8 = NG, K4 = (K + 3) / 4;
#pragma unroll
    for (int g = 0; g < GPT; g++) {
        const int64_t c = tid + (int64_t)g * nt;
        if (c >= NG) continue;
        if (a.dig4) {
            uint32_t w[6];
            digit_words<UT_FMT_INT4>(v[g], 8, sh, w);
#pragma unroll
            for (int p = 0; p < 6; p++) a.dig4[(m * 6 + p) * K8 + c] = w[p];
        }
        if (a.dig8) {
            uint32_t w[3];
            digit_words<UT_FMT_INT8>(v[g], 4, sh, w);
            if (2 * c + 1 < K4 && (K4 & 1) == 0 && ((uintptr_t)a.dig8 & 7) == 0) {
                // both words of the group in one 8-byte store per plane
                uint32_t w2[3];
                digit_words<UT_FMT_INT8>(v[g] + 4, 4, sh, w2);
#pragma unroll
                for (int p = 0; p < 3; p++)
                    *(uint2 *)(a.dig8 + (m * 3 + p) * K4 + 2 * c) = make_uint2(w[p], w2[p]);
            } else {
#pragma unroll
                for (int p = 0; p < 3; p++) a.dig8[(m * 3 + p) * K4 + 2 * c] = w[p];
                if (2 * c + 1 < K4) {
                    digit_words<UT_FMT_INT8>(v[g] + 4, 4, sh, w);
#pragma unroll
                    for (int p = 0; p < 3; p++) a.dig8[(m * 3 + p) * K4 + 2 * c + 1] = w[p];
                }
            }
        }
        if (a.xt) {
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (8 * c + j < K)
                    a.xt[m * K + 8 * c + j] =
                        bad ? 0 : (int32_t)rintf(ldexpf(v[g][j], sh));
        }
    }
}

}  // namespace ut
