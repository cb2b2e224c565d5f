// ut_gemv.hip -- QTensor::matmul on gfx950 (undertow-quant/src/qtensor.rs:
// 281-493 and the kernels it dispatches to, kernels.rs:21-81 /
// avx512.rs:197-267): activation digitisation, the fast skinny GEMV
// (int4 / int8 / f32 weights, 1..4 activation rows per pass) and a generic
// kernel for shapes the fast one does not take.
#include <atomic>
#include "ut_argmax.h"
#include "ut_gemv_core.h"
#include "ut_gemv_mfma.h"
#include "ut_moe.h"
#include "ut_ops.h"
#include "ut_rowdig.h"
#include "ut_sample.h"


namespace ut {

// ------------------------------------------------------- digitisation ---
size_t xdigits_bytes(int64_t M, int64_t K, int flags) {
    size_t b = ((size_t)M * 4 + 255) & ~size_t(255);
    int64_t K8 = (K + 7) / 8, K4 = (K + 3) / 4;
    if (flags & XD_DIG4) b += (((size_t)M * 6 * K8 * 4) + 255) & ~size_t(255);
    if (flags & XD_DIG8) b += (((size_t)M * 3 * K4 * 4) + 255) & ~size_t(255);
    if (flags & XD_XT) b += (((size_t)M * K * 4) + 255) & ~size_t(255);
    return b;
}

XDigits xdigits_view(void *base, int64_t M, int64_t K, int flags) {
    XDigits d;
    d.M = M;
    d.K = K;
    char *p = (char *)base;
    d.exps = (int32_t *)p;
    p += ((size_t)M * 4 + 255) & ~size_t(255);
    int64_t K8 = (K + 7) / 8, K4 = (K + 3) / 4;
    if (flags & XD_DIG4) { d.dig4 = (uint32_t *)p; p += (((size_t)M * 6 * K8 * 4) + 255) & ~size_t(255); }
    if (flags & XD_DIG8) { d.dig8 = (uint32_t *)p; p += (((size_t)M * 3 * K4 * 4) + 255) & ~size_t(255); }
    if (flags & XD_XT) { d.xt = (int32_t *)p; }
    return d;
}

int xdigit_flags_for(int32_t fmt, int64_t K) {
    if (fmt == UT_FMT_INT4) return (K % 32 == 0) ? XD_DIG4 : XD_XT;
    if (fmt == UT_FMT_INT8) return (K % 16 == 0) ? XD_DIG8 : XD_XT;
    return 0;
}

// One workgroup per activation row.  x~ = rint(x * 2^(22-E)) with
// max|x| < 2^E (frexp), so |x~| <= 2^22 and six balanced base-16 digits
// (or three base-256 digits) represent it exactly.
//
// With norm_w set, the row is first rms-normalised exactly as
// undertow-quant/src/lib.rs:91-100 (mean of squares in f64,
// r = 1/sqrt((float)ms + eps), v = (x*r)*w) and the normalised row is what
// gets digitised (and optionally written out as f32): one launch instead of
// a norm kernel plus a digitise kernel per consumer.
constexpr int kRowLds = 16384;  // rows up to this width are staged in LDS


__global__ __launch_bounds__(256) void k_rowdig(RowDigArgs a) {
    extern __shared__ float row[];
    __shared__ double redd[4];
    __shared__ uint32_t redu[4];
    const int64_t m = blockIdx.x;
    if (a.plan_ids && blockIdx.x == gridDim.x - 1) {
        make_plan(a.plan_ids, a.plan_M, a.plan_k, a.plan_E, a.tbl, -1, a.plan, a.err_flag);
        return;
    }
    if (a.slot_count && (int)(m / a.rows_per_slot) >= *a.slot_count) return;
    const int tid = threadIdx.x;
    const int64_t K = a.K;
    const float *xr = a.x + m * a.ldx;
    const bool staged = K <= kRowLds;
    float r = 1.0f;
    if (a.norm_w) {
        double acc = 0.0;
#pragma unroll 8
        for (int64_t i = tid; i < K; i += 256) {
            const double v = (double)xr[i];
            acc += v * v;
        }
        acc = block_reduce(acc, [](double p, double q) { return p + q; }, redd);
        r = 1.0f / sqrtf(__fadd_rn((float)(acc / (double)K), a.eps));
    }
    auto val = [&](int64_t i) -> float {
        return a.norm_w ? __fmul_rn(__fmul_rn(xr[i], r), a.norm_w[i]) : xr[i];
    };
    uint32_t mx = 0;
#pragma unroll 8
    for (int64_t i = tid; i < K; i += 256) {
        const float v = val(i);
        if (staged) row[i] = v;
        if (a.out) a.out[m * a.ldo + i] = v;
        mx = max(mx, __float_as_uint(fabsf(v)));
    }
    if (a.rowmax) {
        mx = 0;
        for (int i = tid; i < a.nparts; i += 256) mx = max(mx, a.rowmax[m * a.nparts + i]);
    }
    mx = block_reduce(mx, [](uint32_t p, uint32_t q) { return p > q ? p : q; }, redu);
    // non-finite rows (|x| bits >= +inf) produce NaN outputs downstream
    const bool bad = mx >= 0x7f800000u;
    int E = 0;
    if (!bad && mx != 0) (void)frexpf(__uint_as_float(mx), &E);
    const int sh = 22 - E;
    if (tid == 0) a.exps[m] = bad ? INT32_MIN : E - 22;
    auto xq = [&](int64_t k) -> int32_t {
        if (bad || k >= K) return 0;
        return (int32_t)rintf(ldexpf(staged ? row[k] : val(k), sh));
    };
    if (a.dig4) {
        const int64_t K8 = (K + 7) / 8;
        for (int64_t c = tid; c < K8; c += 256) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int64_t k = 8 * c + j;
                v[j] = k < K ? (staged ? row[k] : val(k)) : 0.0f;
            }
            uint32_t w[6];
            digit_words<UT_FMT_INT4>(v, 8, bad ? INT32_MIN : sh, w);
#pragma unroll
            for (int p = 0; p < 6; p++) a.dig4[(m * 6 + p) * K8 + c] = w[p];
        }
    }
    if (a.dig8) {
        const int64_t K4 = (K + 3) / 4;
        for (int64_t c = tid; c < K4; c += 256) {
            float v[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int64_t k = 4 * c + j;
                v[j] = k < K ? (staged ? row[k] : val(k)) : 0.0f;
            }
            uint32_t w[3];
            digit_words<UT_FMT_INT8>(v, 4, bad ? INT32_MIN : sh, w);
#pragma unroll
            for (int p = 0; p < 3; p++) a.dig8[(m * 3 + p) * K4 + c] = w[p];
        }
    }
    if (a.xt) {
        for (int64_t k = tid; k < K; k += 256) a.xt[m * K + k] = xq(k);
    }
}

// The same work with the row held in registers: thread t owns the 8-column
// groups t, t + T, ... (GPT of them), all loads of the row are issued before
// the first use, and every digit word is formed from the owner's registers.
// One global round trip per row instead of one per 256 columns.
//

template <int GPT>
__global__ __launch_bounds__(1024) void k_rowdig_reg(RowDigArgs a) {
    __shared__ double redd[16];
    __shared__ uint32_t redu[16];
    const int64_t m = blockIdx.x;
    if (a.plan_ids && blockIdx.x == gridDim.x - 1) {
        make_plan(a.plan_ids, a.plan_M, a.plan_k, a.plan_E, a.tbl, -1, a.plan, a.err_flag);
        return;
    }
    if (a.slot_count && (int)(m / a.rows_per_slot) >= *a.slot_count) return;
    const int tid = threadIdx.x, nt = blockDim.x;
    const int64_t K = a.K;
    const float *xr = a.x + m * a.ldx;
    const bool vec = ((uintptr_t)xr & 15) == 0 &&
                     (!a.norm_w || ((uintptr_t)a.norm_w & 15) == 0);
    auto load8 = [&](const float *src, int64_t c, float (&v)[8]) {
        const int64_t k0 = 8 * c;
        if (vec && k0 + 8 <= K) {
            const float4 p = *(const float4 *)(src + k0), q = *(const float4 *)(src + k0 + 4);
            v[0] = p.x; v[1] = p.y; v[2] = p.z; v[3] = p.w;
            v[4] = q.x; v[5] = q.y; v[6] = q.z; v[7] = q.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = k0 + j < K ? src[k0 + j] : 0.0f;
        }
    };
    const int64_t NG = (K + 7) / 8;
    float v[GPT][8], wv[GPT][8];
#pragma unroll
    for (int g = 0; g < GPT; g++) {
        const int64_t c = tid + (int64_t)g * nt;
        if (c < NG) {
            load8(xr, c, v[g]);
            if (a.norm_w) load8(a.norm_w, c, wv[g]);
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) v[g][j] = 0.0f, wv[g][j] = 0.0f;
        }
    }
    rowdig_body<GPT>(a, m, v, wv, redd, redu);
}


constexpr int64_t kRowRegCols = 4 * 8 * 1024;  // widest row the register kernel takes

// The embedding lookup and the first layer's input norm in one launch: row
// m's values are k_embed's (0 + (1 * scale[id]) * q, the reference's
// add_scaled_row into zeros), formed in the registers of the thread that
// owns their 8-column group, then the row digitiser's body, which also
// stores the looked-up row to a.raw (the residual stream).
__global__ __launch_bounds__(1024) void k_rowdig_emb(RowDigArgs a, int32_t fmt,
                                                     const uint8_t *__restrict__ payload,
                                                     const float *__restrict__ scales,
                                                     int64_t row_bytes,
                                                     const int32_t *__restrict__ ids) {
    __shared__ double redd[16];
    __shared__ uint32_t redu[16];
    const int64_t m = blockIdx.x;
    const int tid = threadIdx.x;
    const int64_t NG = a.K / 8, c = tid;
    const int64_t id = ids[m];
    const uint8_t *row = payload + id * row_bytes;
    const float f = fmt == UT_FMT_F32 ? 1.0f : __fmul_rn(1.0f, scales[id]);
    float v[1][8], wv[1][8];
    if (c < NG) {
        const float4 w0 = *(const float4 *)(a.norm_w + 8 * c), w1 = *(const float4 *)(a.norm_w + 8 * c + 4);
        wv[0][0] = w0.x; wv[0][1] = w0.y; wv[0][2] = w0.z; wv[0][3] = w0.w;
        wv[0][4] = w1.x; wv[0][5] = w1.y; wv[0][6] = w1.z; wv[0][7] = w1.w;
#pragma unroll
        for (int j = 0; j < 8; j++) v[0][j] = __fadd_rn(0.0f, __fmul_rn(f, code_at(fmt, row, 8 * c + j)));
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++) v[0][j] = 0.0f, wv[0][j] = 0.0f;
    }
    rowdig_body<1, true>(a, m, v, wv, redd, redu);
}

// The MTP module's input rows (mtp.rs: cat = [enorm(embed(id)) | hnorm(h)])
// in one launch of two workgroups per row, one per half: the embedding row
// as k_embed forms it (0 + (1 * scale[id]) * q), or the hidden row; each
// rms-normalised (thread t sums its elements t, t + 1024, ... in f64, the
// waves by the DPP butterfly and then in wave order), written to cat
// [rows][2H], and the half's max|v| left as a partial maximum (float bits,
// [rows][2]) from which eh_proj digitises the row while staging it.
__global__ __launch_bounds__(1024) void k_mtp_input(int32_t fmt, const uint8_t *__restrict__ payload,
                                                    const float *__restrict__ scales,
                                                    int64_t row_bytes,
                                                    const int32_t *__restrict__ ids,
                                                    const float *__restrict__ hidden, int64_t H,
                                                    const float *__restrict__ enorm,
                                                    const float *__restrict__ hnorm, float eps,
                                                    float *__restrict__ cat,
                                                    uint32_t *__restrict__ vmax) {
    __shared__ double redd[16];
    __shared__ uint32_t redu[16];
    constexpr int PT = 8;  // elements per thread (H <= 8192)
    const int half = blockIdx.x;
    const int64_t m = blockIdx.y;
    const int tid = threadIdx.x, nt = blockDim.x;
    const float *w = half ? hnorm : enorm;
    float v[PT];
    double acc = 0.0;
    if (half == 0) {
        const int64_t id = ids[m];
        const uint8_t *row = payload + id * row_bytes;
        const float f = fmt == UT_FMT_F32 ? 1.0f : __fmul_rn(1.0f, scales[id]);
#pragma unroll
        for (int k = 0; k < PT; k++) {
            const int64_t i = tid + (int64_t)k * nt;
            v[k] = i < H ? __fadd_rn(0.0f, __fmul_rn(f, code_at(fmt, row, i))) : 0.0f;
        }
    } else {
        const float *hr = hidden + m * H;
#pragma unroll
        for (int k = 0; k < PT; k++) {
            const int64_t i = tid + (int64_t)k * nt;
            v[k] = i < H ? hr[i] : 0.0f;
        }
    }
#pragma unroll
    for (int k = 0; k < PT; k++) acc += (double)v[k] * (double)v[k];
    acc = wide_reduce(acc, [](double p, double q) { return p + q; }, redd);
    const float r = 1.0f / sqrtf(__fadd_rn((float)(acc / (double)H), eps));
    uint32_t mx = 0;
    float *o = cat + m * 2 * H + half * H;
#pragma unroll
    for (int k = 0; k < PT; k++) {
        const int64_t i = tid + (int64_t)k * nt;
        if (i < H) {
            const float x = __fmul_rn(__fmul_rn(v[k], r), w[i]);
            o[i] = x;
            mx = max(mx, __float_as_uint(fabsf(x)));
        }
    }
    mx = wide_reduce(mx, [](uint32_t p, uint32_t q) { return p > q ? p : q; }, redu);
    if (tid == 0) vmax[m * 2 + half] = mx;
}

bool mtp_input_ok(int64_t H) { return H % 4 == 0 && H <= 8 * 1024; }

int32_t launch_mtp_input(ut_ctx *ctx, const ut_qtensor *emb, const int32_t *ids,
                         const float *hidden, int64_t rows, int64_t H, const float *enorm,
                         const float *hnorm, float eps, float *cat, uint32_t *vmax) {
    if (!mtp_input_ok(H) || emb->in_dim != H) {
        set_error(ctx, "mtp_input: hidden %lld unsupported", (long long)H);
        return UT_ERR_ARG;
    }
    if (rows <= 0) return UT_OK;
    int64_t nt = (H + 7) / 8;
    nt = (nt + 63) / 64 * 64;
    int tok = timing_begin(ctx, "mtp_input");
    hipLaunchKernelGGL(k_mtp_input, dim3(2, (unsigned)rows), dim3((unsigned)nt), 0, ctx->stream,
                       emb->fmt, (const uint8_t *)emb->payload, emb->scales, emb->row_bytes, ids,
                       hidden, H, enorm, hnorm, eps, cat, vmax);
    timing_end(ctx, tok);
    return launch_check(ctx, "k_mtp_input");
}

bool embed_norm_ok(const ut_qtensor *emb, int64_t K, const float *x, const float *norm_w) {
    return K % 8 == 0 && K <= 8 * 1024 && emb->in_dim == K && ((uintptr_t)x & 15) == 0 &&
           ((uintptr_t)norm_w & 15) == 0;
}

int32_t launch_embed_norm(ut_ctx *ctx, const ut_qtensor *emb, const int32_t *ids, int64_t rows,
                          float *x, int64_t ldx, const NormNext &nx) {
    const int64_t K = emb->in_dim;
    if (!embed_norm_ok(emb, K, x, nx.norm_w) || ldx % 4 != 0) {
        set_error(ctx, "embed_norm: rows of a multiple of 8 columns, at most 8192, 16-byte aligned");
        return UT_ERR_ARG;
    }
    if (rows <= 0) return UT_OK;
    RowDigArgs a{};
    a.K = K;
    a.norm_w = nx.norm_w;
    a.eps = nx.eps;
    a.out = nx.normed;
    a.ldo = nx.ldn;
    a.exps = nx.nd.exps;
    a.dig4 = (nx.flags & XD_DIG4) ? nx.nd.dig4 : nullptr;
    a.dig8 = (nx.flags & XD_DIG8) ? nx.nd.dig8 : nullptr;
    a.xt = (nx.flags & XD_XT) ? nx.nd.xt : nullptr;
    a.raw = x;
    a.ldr = ldx;
    const unsigned threads = (unsigned)((K / 8 + 63) / 64 * 64);
    int tok = timing_begin(ctx, "embed_norm");
    hipLaunchKernelGGL(k_rowdig_emb, dim3((unsigned)rows), dim3(threads), 0, ctx->stream, a,
                       emb->fmt, (const uint8_t *)emb->payload, emb->scales, emb->row_bytes, ids);
    timing_end(ctx, tok);
    return launch_check(ctx, "k_rowdig_emb");
}

// After the kv_a / q_a pair GEMV's split-K pass (kv_a rows first, then
// q_a): workgroup m < M sums row m's q_a partials, rms-normalises and
// digitises them for q_b (the row digitiser's body); workgroup M + m sums
// row m's kv_a partials into LDS and appends them to the cache.  The
// partials are exact integer totals, so these sums equal the split-K sum
// kernel's values bit for bit; one launch replaces three.
struct MlaPreArgs {
    const int64_t *part;
    int ks;
    int64_t O, O1;  // pair rows, kv_a rows
    const int32_t *exps;
    const float *kv_scales, *q_scales;
    int M;
    RowDigArgs qa;  // K = q_lora_rank, norm_w = q_a_norm
    // set: q_a's rows go here as summed (un-normalised) and qa is unused
    // (the q_b GEMV normalises them while staging)
    float *qa_raw;
    int64_t L, P;
    const float *kv_norm;
    float *latent, *krot;
    __bf16 *kc;
    PosRef pos;
    const float2 *table;
};

// Exact sum over the ks partials of element i (z-stride zs), 16 loads in
// flight per call.
__device__ __forceinline__ int64_t splitk_total(const int64_t *__restrict__ part, int ks,
                                                int64_t zs, int64_t i) {
    int64_t S = 0;
    for (int z0 = 0; z0 < ks; z0 += 16) {
        int64_t t[16];
#pragma unroll
        for (int u = 0; u < 16; u++) t[u] = z0 + u < ks ? part[(z0 + u) * zs + i] : 0;
#pragma unroll
        for (int u = 0; u < 16; u++) S += t[u];
    }
    return S;
}

__global__ __launch_bounds__(1024) void k_mla_pre(MlaPreArgs a) {
    __shared__ double redd[16];
    __shared__ uint32_t redu[16];
    __shared__ double red4[16];
    __shared__ float sc[kMlaPreMaxComp > 2048 ? kMlaPreMaxComp : 2048];
    const int tid = threadIdx.x;
    const int64_t zs = (int64_t)a.M * a.O;
    const bool qrow = (int)blockIdx.x < a.M;
    const int64_t m = qrow ? blockIdx.x : blockIdx.x - a.M;
    // the row's values into LDS (every thread, coalesced partial reads)
    const int64_t n = qrow ? a.qa.K : a.O1, off = m * a.O + (qrow ? a.O1 : 0);
    const float *scl = qrow ? a.q_scales : a.kv_scales;
    for (int64_t i = tid; i < n; i += blockDim.x)
        sc[i] = int_total_to_f32(splitk_total(a.part, a.ks, zs, off + i), a.exps[m], ld_global_f32(scl + i));
    if (qrow && a.qa_raw) {
        for (int64_t i = tid; i < n; i += blockDim.x) a.qa_raw[m * n + i] = sc[i];
        return;
    }
    __syncthreads();
    if (qrow) {
        const int64_t K = a.qa.K, NG = (K + 7) / 8;
        float v[1][8], wv[1][8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int64_t col = 8 * tid + j;
            const bool in = tid < NG && col < K;
            v[0][j] = in ? sc[col] : 0.0f;
            wv[0][j] = in ? a.qa.norm_w[col] : 0.0f;
        }
        rowdig_body<1>(a.qa, m, v, wv, redd, redu);
    } else {
        kv_append_row(sc, a.L, a.P, a.kv_norm, a.qa.eps, a.latent, a.krot, a.kc, a.pos.get() + m,
                      a.table, red4);
    }
}

bool mla_pre_ok(int64_t M, int64_t q_lora, int64_t L, int64_t P) {
    return M >= 1 && M <= 4 && q_lora <= 8 * 256 && L + P <= kMlaPreMaxComp;
}

int32_t launch_mla_pre(ut_ctx *ctx, const SplitKPartials &pp, int64_t O1, const int32_t *exps,
                       const float *kv_scales, const float *q_scales, int64_t M, int64_t q_lora,
                       const float *q_norm, float eps, float *qa_n, const XDigits &qd, int flags,
                       int64_t L, int64_t P, const float *kv_norm, float *latent, float *krot,
                       __bf16 *kc, int64_t pos_base, const float2 *table, float *qa_raw) {
    if (!mla_pre_ok(M, q_lora, L, P) || pp.ks < 1 || !pp.part || O1 != L + P) {
        set_error(ctx, "mla_pre: unsupported shape");
        return UT_ERR_ARG;
    }
    MlaPreArgs a{};
    a.part = pp.part;
    a.ks = pp.ks;
    a.O = pp.O;
    a.O1 = O1;
    a.exps = exps;
    a.kv_scales = kv_scales;
    a.q_scales = q_scales;
    a.M = (int)M;
    a.qa.K = q_lora;
    a.qa.norm_w = q_norm;
    a.qa.eps = eps;
    a.qa.out = qa_n;
    a.qa.ldo = q_lora;
    a.qa.exps = qd.exps;
    a.qa.dig4 = (flags & XD_DIG4) ? qd.dig4 : nullptr;
    a.qa.dig8 = (flags & XD_DIG8) ? qd.dig8 : nullptr;
    a.qa.xt = (flags & XD_XT) ? qd.xt : nullptr;
    a.L = L;
    a.P = P;
    a.kv_norm = kv_norm;
    a.latent = latent;
    a.krot = krot;
    a.kc = kc;
    a.pos = pos_ref(ctx, pos_base);
    a.table = table;
    a.qa_raw = qa_raw;
    int tok = timing_begin(ctx, "mla_pre");
    hipLaunchKernelGGL(k_mla_pre, dim3((unsigned)(2 * M)), dim3(1024), 0, ctx->stream, a);
    timing_end(ctx, tok);
    return launch_check(ctx, "k_mla_pre");
}



static int32_t launch_rowdig(ut_ctx *ctx, const RowDigArgs &a, int64_t M, const char *name) {
    if (M <= 0) return UT_OK;
    const dim3 grid((unsigned)(M + (a.plan_ids ? 1 : 0)));
    int tok = timing_begin(ctx, name);
    if (a.K <= kRowRegCols) {
        const int64_t NG = (a.K + 7) / 8;
        const int gpt = NG <= 1024 ? 1 : NG <= 2048 ? 2 : 4;
        int64_t nt = (NG + gpt - 1) / gpt;
        nt = (nt + 63) / 64 * 64;
        // the plan workgroup needs at least the threads make_plan assumes
        if (a.plan_ids && nt < 256) nt = 256;
        switch (gpt) {
        case 1: hipLaunchKernelGGL(k_rowdig_reg<1>, grid, dim3((unsigned)nt), 0, ctx->stream, a); break;
        case 2: hipLaunchKernelGGL(k_rowdig_reg<2>, grid, dim3((unsigned)nt), 0, ctx->stream, a); break;
        default: hipLaunchKernelGGL(k_rowdig_reg<4>, grid, dim3((unsigned)nt), 0, ctx->stream, a); break;
        }
    } else {
        const size_t shmem = a.K <= kRowLds ? (size_t)a.K * 4 : 0;
        hipLaunchKernelGGL(k_rowdig, grid, dim3(256), shmem, ctx->stream, a);
    }
    timing_end(ctx, tok);
    return launch_check(ctx, "k_rowdig");
}

int32_t launch_digitize(ut_ctx *ctx, const float *x, int64_t ldx, int64_t M, int64_t K,
                        const uint32_t *rowmax_bits, XDigits xd, int flags) {
    return launch_digitize_parts(ctx, x, ldx, M, K, rowmax_bits, 1, xd, flags);
}

int32_t launch_digitize_parts(ut_ctx *ctx, const float *x, int64_t ldx, int64_t M, int64_t K,
                              const uint32_t *rowmax_parts, int32_t nparts, XDigits xd,
                              int flags) {
    return launch_digitize_slots(ctx, x, ldx, M, K, rowmax_parts, nparts, xd, flags, nullptr, 1);
}

int32_t launch_digitize_slots(ut_ctx *ctx, const float *x, int64_t ldx, int64_t M, int64_t K,
                              const uint32_t *rowmax_parts, int32_t nparts, XDigits xd,
                              int flags, const int32_t *slot_count, int rows_per_slot) {
    RowDigArgs a{};
    a.x = x;
    a.ldx = ldx;
    a.K = K;
    a.rowmax = rowmax_parts;
    a.nparts = nparts;
    a.slot_count = slot_count;
    a.rows_per_slot = rows_per_slot;
    a.exps = xd.exps;
    a.dig4 = (flags & XD_DIG4) ? xd.dig4 : nullptr;
    a.dig8 = (flags & XD_DIG8) ? xd.dig8 : nullptr;
    a.xt = (flags & XD_XT) ? xd.xt : nullptr;
    return launch_rowdig(ctx, a, M, "digitize");
}

int32_t launch_digitize_plan(ut_ctx *ctx, const float *x, int64_t M, int64_t K, XDigits xd,
                             int flags, const int32_t *ids, int k, int64_t E,
                             const void *const *tbl, MoePlan plan, int32_t *err_flag) {
    RowDigArgs a{};
    a.x = x;
    a.ldx = K;
    a.K = K;
    a.exps = xd.exps;
    a.dig4 = (flags & XD_DIG4) ? xd.dig4 : nullptr;
    a.dig8 = (flags & XD_DIG8) ? xd.dig8 : nullptr;
    a.xt = (flags & XD_XT) ? xd.xt : nullptr;
    a.plan_ids = ids;
    a.plan_M = (int)M;
    a.plan_k = k;
    a.plan_E = (int)E;
    a.tbl = tbl;
    a.plan = plan;
    a.err_flag = err_flag;
    return launch_rowdig(ctx, a, M, "digitize_plan");
}

int32_t launch_rmsnorm_digitize(ut_ctx *ctx, const float *x, int64_t ldx, int64_t M, int64_t K,
                                const float *w, float eps, float *out, int64_t ldo, XDigits xd,
                                int flags) {
    RowDigArgs a{};
    a.x = x;
    a.ldx = ldx;
    a.K = K;
    a.norm_w = w;
    a.eps = eps;
    a.out = out;
    a.ldo = ldo;
    a.exps = xd.exps;
    a.dig4 = (flags & XD_DIG4) ? xd.dig4 : nullptr;
    a.dig8 = (flags & XD_DIG8) ? xd.dig8 : nullptr;
    a.xt = (flags & XD_XT) ? xd.xt : nullptr;
    return launch_rowdig(ctx, a, M, "rmsnorm_digitize");
}

// --------------------------------------------------------- fast GEMV ---
// Rows [0, O1) come from weight w, rows [O1, O) from w2 (same format, K and
// row bytes), written to out / out2: two projections of one activation
// (e.g. kv_a and q_a) in one launch.
struct PlainArgs {
    const uint8_t *w, *w2;
    const float *scales, *scales2;
    int64_t O, O1, K, row_bytes;
    XSrc x;
    const int32_t *exps;
    float *out, *out2;
    int64_t ldo, ldo2;
    int accumulate;
    // split-K over blockIdx.z (ks > 1): columns [z*kslice, (z+1)*kslice),
    // partial totals to part[(z*M + m)*O + row]; k_gemv_splitk_sum finishes
    int ks;
    int64_t kslice;
    int64_t *part;
    // x.dig == nullptr for int weights: the row shifts come from partial
    // maxima xmax [M][nxmax]; workgroup 0 records the exponents in exps
    const uint32_t *xmax;
    int nxmax;
    // optional: the launch that finishes the rows leaves argmax partials
    // (k_gemv / k_gemv_mfma_i8 unsplit: one per workgroup; split: the sum's)
    ArgmaxParts am;
    // optional (k_gemv NORM): one more workgroup appends a finished kv_a
    // row to the latent cache (kv_append_row) beside the GEMV's
    KvAppendArgs kv;
};

__device__ __forceinline__ const uint8_t *plain_row(const PlainArgs &a, int64_t row) {
    return row < a.O1 ? a.w + row * a.row_bytes : a.w2 + (row - a.O1) * a.row_bytes;
}
__device__ __forceinline__ float plain_scale(const PlainArgs &a, int64_t row) {
    return ld_global_f32(row < a.O1 ? a.scales + row : a.scales2 + (row - a.O1));
}
__device__ __forceinline__ float *plain_out(const PlainArgs &a, int64_t m, int64_t row) {
    return row < a.O1 ? a.out + m * a.ldo + row : a.out2 + m * a.ldo2 + (row - a.O1);
}

// 32 output rows per workgroup (R = 2 rows per lane: registers for three or
// four workgroups per CU; four rows per lane at M = 2 held two or three and
// measured slower): wave w, row group g, slot r -> row blockIdx.x*16R +
// w*4R + g*R + r.  Weight steps in flight: every step of a short row at
// M = 1, two at M = 2, the core's default above.
template <int M> constexpr int plain_rows() { return 2; }
template <int M> constexpr int plain_depth() { return M == 1 ? 4 : M == 2 ? 2 : gemv_depth<M>(); }
__host__ __device__ constexpr int plain_rows_rt(int) { return 16 * 2; }

// NORM: x is one un-normalised row, normalised while staged (XSrc::nw).
// The kv appends' workgroups first in the normalising GEMV's grid (config-4
// one-row q_b 11.0 -> 10.3 us), or last.
#ifndef UT_KV_APPEND_FIRST
#define UT_KV_APPEND_FIRST 1
#endif
constexpr int kGemvNormCols = 2048;
template <int FMT, int M, bool NORM = false>
__global__ __launch_bounds__(kGemvThreads) void k_gemv(PlainArgs a) {
    constexpr int R = plain_rows<M>();
    // bx: this workgroup's row tile
    int bx = (int)blockIdx.x;
    if constexpr (NORM) {
        // M more workgroups append the M kv_a rows (row m at pos + m): the
        // grid's first (UT_KV_APPEND_FIRST), so their chain of reductions
        // runs beside the tiles instead of after them, or its last
        if (a.kv.comp) {
            const int m = UT_KV_APPEND_FIRST ? bx : bx - ((int)gridDim.x - M);
            if (m >= 0 && m < M) {
                __shared__ double red4[4];
                const KvAppendArgs &k = a.kv;
                kv_append_row(k.comp + m * (k.L + k.P), k.L, k.P, k.w, k.eps, k.latent, k.krot,
                              k.kc, k.pos.get() + m, k.table, red4);
                return;
            }
            if (UT_KV_APPEND_FIRST) bx -= M;
        }
    }
    __shared__ __attribute__((aligned(16))) uint32_t lds[kLdsWords];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, s = lane & 15;
    const int64_t row0 = (int64_t)bx * (16 * R) + wave * (4 * R) + g * R;
    const uint8_t *rows[R];
#pragma unroll
    for (int r = 0; r < R; r++) rows[r] = plain_row(a, row0 + r < a.O ? row0 + r : a.O - 1);
    XSrc xs = a.x;
    int32_t exl[M];
    const int64_t kb = a.ks > 1 ? (int64_t)blockIdx.z * a.kslice : 0;
    const int64_t ke = a.ks > 1 ? (kb + a.kslice < a.K ? kb + a.kslice : a.K) : a.K;
    // x's row shifts from the producer's partial maxima (xmax): their loads
    // go out first; on the one-chunk path the reduction runs inside the
    // staging, after the first weight loads (prep)
    __shared__ uint32_t redm[4 * M];
    ut_u32x4 pv[M];
    const bool late = FMT != UT_FMT_F32 && a.xmax && gemv_one_chunk<FMT, M>(kb, ke);
    auto shifts = [&](int32_t (&shl)[4]) {
        int32_t sh[M];
        rowmax_reduce<M>(pv, sh, redm);
#pragma unroll
        for (int m = 0; m < M; m++) {
            shl[m] = sh[m];
            exl[m] = sh[m] == INT32_MIN ? INT32_MIN : -sh[m];
        }
        if (bx == 0 && blockIdx.z == 0 && tid < M)
            const_cast<int32_t *>(a.exps)[tid] = tid == 0 ? exl[0] : tid == 1 ? exl[M > 1 ? 1 : 0]
                                                : tid == 2 ? exl[M > 2 ? 2 : 0] : exl[M > 3 ? 3 : 0];
    };
    if constexpr (FMT != UT_FMT_F32) {
        if (a.xmax) {
            rowmax_load<M>(a.xmax, a.nxmax, pv);
            if (!late) shifts(xs.sh);
        } else if (!NORM) {
#pragma unroll
            for (int m = 0; m < M; m++) exl[m] = a.exps[m];
        }
    }
    auto prep = [&](int32_t (&shl)[4]) {
        if constexpr (FMT != UT_FMT_F32) {
            if (late) shifts(shl);
            // normalised while staged: the staging found the rows' shifts
            if constexpr (NORM)
#pragma unroll
                for (int m = 0; m < M; m++)
                    exl[m] = shl[m] == INT32_MIN ? INT32_MIN : -shl[m];
        }
    };
    CoreOut<FMT, M, R> res;
    if (!NORM && a.ks > 1) {
        gemv_core<FMT, M, R, plain_depth<M>()>(rows, a.K, xs, lds, res, kb, ke, prep);
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int m = 0; m < M; m++) {
                const int64_t row = row0 + r;
                if (s == 4 * r + m && row < a.O)
                    a.part[((int64_t)blockIdx.z * M + m) * a.O + row] =
                        FMT == UT_FMT_F32 ? (int64_t)__float_as_uint(res.F[r][m]) : res.S[r][m];
            }
        return;
    }
    // the normalising staging holds its row's groups in registers: rows of
    // at most kGemvNormCols columns (one group per thread)
    constexpr int KC = NORM ? gemv_chunk_cols<FMT, M, kGemvNormCols>() : gemv_chunk_cols<FMT, M>();
    // one normalised row is short: six steps in flight (all of a 1,536-column
    // int8 row, the q_a width: q_b 11.3 -> 10.9 us at config 4; at two rows
    // six made it 12.7 -> 14.0 us)
    constexpr int DEPTH = NORM && M == 1 ? 6 : plain_depth<M>();
    gemv_core<FMT, M, R, DEPTH, KC, false, decltype(prep) &, NoMid, NORM>(
        rows, a.K, xs, lds, res, 0, -1, prep);
    Best bm[M];
#pragma unroll
    for (int m = 0; m < M; m++) bm[m] = Best{0.0f, -1};
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int m = 0; m < M; m++) {
            const int64_t row = row0 + r;
            if (s == 4 * r + m && row < a.O) {
                const float v = FMT == UT_FMT_F32
                                    ? res.F[r][m]
                                    : int_total_to_f32(res.S[r][m], exl[m], plain_scale(a, row));
                float *o = plain_out(a, m, row);
                const float nv = a.accumulate ? __fadd_rn(*o, v) : v;
                *o = nv;
                argmax_offer(bm[m], nv, row);
            }
        }
    if (a.am.v) argmax_parts_store<M>(a.am, bm, bx);
}

// int8 weights at 3..4 activation rows on the matrix cores
// (mfma_gemv_i8): 64 * TW output rows per workgroup, wave w's TW tiles of
// 16 rows at blockIdx.x * 64TW + 16TW w + 16t; the same split-K partials,
// epilogue and partial-maxima path (F32X: x digitised while staged) as
// k_gemv, and the same totals, so the outputs are bit-identical to its.
// UT_GEMV_I8_MFMA_MIN_M: the fewest rows that take it.
#ifndef UT_GEMV_I8_MFMA_MIN_M
#define UT_GEMV_I8_MFMA_MIN_M 3
#endif
#ifndef UT_GEMV_I8_MFMA_TW
#define UT_GEMV_I8_MFMA_TW 1
#endif
#ifndef UT_GEMV_I8_MFMA_DEPTH
#define UT_GEMV_I8_MFMA_DEPTH 2
#endif
#ifndef UT_GEMV_I8_MFMA_SPLIT_FILL
#define UT_GEMV_I8_MFMA_SPLIT_FILL 0
#endif
#ifndef UT_GEMV_I8_MFMA_KC4
#define UT_GEMV_I8_MFMA_KC4 2048
#endif
template <int M> constexpr int gemv_i8_mfma_tw() { return UT_GEMV_I8_MFMA_TW; }
template <int M> constexpr int gemv_i8_mfma_kc() { return M <= 2 ? 4096 : UT_GEMV_I8_MFMA_KC4; }
template <int M> constexpr int gemv_i8_mfma_depth() { return UT_GEMV_I8_MFMA_DEPTH; }

template <int M, bool F32X, int TW = gemv_i8_mfma_tw<M>()>
__global__ __launch_bounds__(kGemvThreads) void k_gemv_mfma_i8(PlainArgs a) {
    constexpr int KC = gemv_i8_mfma_kc<M>();
    __shared__ __attribute__((aligned(16))) uint8_t lds[mfma_i8_lds_bytes<M, KC>()];
    __shared__ __attribute__((aligned(16))) uint8_t wareas[4 * TW * kMfmaI8WaveAreaBytes];
    __shared__ uint32_t redm[4 * M];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, s = lane & 15;
    const int64_t rowbase = (int64_t)blockIdx.x * (64 * TW) + wave * (16 * TW);
    // load rows: tile w, instruction r -> row 4r + lane / 16 of the tile
    const uint8_t *lrows[TW][4];
#pragma unroll
    for (int w = 0; w < TW; w++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int64_t row = rowbase + 16 * w + 4 * r + g;
            lrows[w][r] = plain_row(a, row < a.O ? row : a.O - 1);
        }
    const int64_t kb = a.ks > 1 ? (int64_t)blockIdx.z * a.kslice : 0;
    const int64_t ke = a.ks > 1 ? (kb + a.kslice < a.K ? kb + a.kslice : a.K) : a.K;
    int32_t exl[M];
    ut_u32x4 pv[M];
    if constexpr (F32X) {
        rowmax_load<M>(a.xmax, a.nxmax, pv);
    } else {
#pragma unroll
        for (int m = 0; m < M; m++) exl[m] = a.exps[m];
    }
    auto prep = [&](int32_t (&shl)[4]) {
        if constexpr (F32X) {
            int32_t sh[M];
            rowmax_reduce<M>(pv, sh, redm);
#pragma unroll
            for (int m = 0; m < M; m++) {
                shl[m] = sh[m];
                exl[m] = sh[m] == INT32_MIN ? INT32_MIN : -sh[m];
            }
            if (blockIdx.x == 0 && blockIdx.z == 0 && tid < M)
                const_cast<int32_t *>(a.exps)[tid] = tid == 0 ? exl[0] : tid == 1 ? exl[M > 1 ? 1 : 0]
                                                    : tid == 2 ? exl[M > 2 ? 2 : 0] : exl[M > 3 ? 3 : 0];
        }
    };
    CoreOut<UT_FMT_INT4, M, 4> res[TW];
    mfma_gemv_i8<M, KC, TW, gemv_i8_mfma_depth<M>(), F32X>(
        lrows, kb, ke, a.x.dig, a.x.KW, a.x.xf, a.x.ldx, lds,
        wareas + wave * TW * kMfmaI8WaveAreaBytes, res, prep);
    Best bm[M];
#pragma unroll
    for (int m = 0; m < M; m++) bm[m] = Best{0.0f, -1};
#pragma unroll
    for (int w = 0; w < TW; w++)
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int m = 0; m < M; m++) {
                const int64_t row = rowbase + 16 * w + 4 * g + r;
                if (s != 4 * r + m || row >= a.O) continue;
                if (a.ks > 1) {
                    a.part[((int64_t)blockIdx.z * M + m) * a.O + row] = res[w].S[r][m];
                } else {
                    const float v = int_total_to_f32(res[w].S[r][m], exl[m], plain_scale(a, row));
                    float *o = plain_out(a, m, row);
                    const float nv = a.accumulate ? __fadd_rn(*o, v) : v;
                    *o = nv;
                    argmax_offer(bm[m], nv, row);
                }
            }
    if (a.ks == 1 && a.am.v) argmax_parts_store<M>(a.am, bm, blockIdx.x);
}

// int8 weights, M <= 4 activation rows (digit planes), rows whose K is
// split inside the workgroup instead of across workgroups: a workgroup
// takes 4 output rows, lane group g (16 lanes) of wave w the quarter w of
// row g's columns, every 256-column step of the quarter in flight at once
// (K <= 8192, K % 1024 == 0).  Per lane the exact plane sums of its 16
// columns per step, the lane total S = sum_p acc_p 256^p in int64, summed
// over the 16 lanes and then over the four quarters: the exact integer
// total of the row, so the output equals the split-K GEMV's bit for bit,
// and the rows come out finished (no partials, no sum launch).  Rows
// [0, O1) of w, [O1, O) of w2 (PlainArgs), activations a.x.dig, exponents
// a.exps[m].
constexpr int kRowSplitMaxSteps = 8;
template <int M>
__global__ __launch_bounds__(kGemvThreads) void k_gemv_i8_rowsplit(PlainArgs a) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, s = lane & 15;
    const int64_t row = (int64_t)blockIdx.x * 4 + g;
    const uint8_t *wr = plain_row(a, row < a.O ? row : a.O - 1);
    const int64_t kq = a.K / 4;
    const int nst = (int)(kq / 256);
    const int64_t c0 = (int64_t)wave * kq + 16 * s;
    uint4 w[kRowSplitMaxSteps];
#pragma unroll
    for (int u = 0; u < kRowSplitMaxSteps; u++)
        if (u < nst) w[u] = ld_weights(wr + c0 + 256 * u);
    int32_t acc[M][3];
#pragma unroll
    for (int m = 0; m < M; m++) acc[m][0] = acc[m][1] = acc[m][2] = 0;
#pragma unroll
    for (int u = 0; u < kRowSplitMaxSteps; u++) {
        if (u >= nst) continue;
        const int64_t wd = (c0 + 256 * u) / 4;
#pragma unroll
        for (int m = 0; m < M; m++)
#pragma unroll
            for (int p = 0; p < 3; p++) {
                const uint4 xv = ld_global<uint4>(a.x.dig + (int64_t)(m * 3 + p) * a.x.KW + wd);
                int t = acc[m][p];
                t = __builtin_amdgcn_sdot4((int)w[u].x, (int)xv.x, t, false);
                t = __builtin_amdgcn_sdot4((int)w[u].y, (int)xv.y, t, false);
                t = __builtin_amdgcn_sdot4((int)w[u].z, (int)xv.z, t, false);
                t = __builtin_amdgcn_sdot4((int)w[u].w, (int)xv.w, t, false);
                acc[m][p] = t;
            }
    }
    __shared__ int64_t part[4][4][M];
#pragma unroll
    for (int m = 0; m < M; m++) {
        int64_t t = ((int64_t)acc[m][2] * 256 + acc[m][1]) * 256 + acc[m][0];
#pragma unroll
        for (int off = 8; off >= 1; off >>= 1) t += shfl_xor_i64(t, off);
        if (s == 0) part[wave][g][m] = t;
    }
    __syncthreads();
    const int gr = tid & 3, m = tid >> 2;
    const int64_t r = (int64_t)blockIdx.x * 4 + gr;
    if (m < M && r < a.O) {
        const int64_t S = part[0][gr][m] + part[1][gr][m] + part[2][gr][m] + part[3][gr][m];
        const float v = int_total_to_f32(S, a.exps[m], plain_scale(a, r));
        float *o = plain_out(a, m, r);
        *o = a.accumulate ? __fadd_rn(*o, v) : v;
    }
}

static bool fast_ok(const ut_qtensor *w);

bool gemv_rowsplit_ok(const GemvArgs &ga) {
    const ut_qtensor *w = ga.w;
    if (!w || w->fmt != UT_FMT_INT8 || ga.M < 1 || ga.M > 2 || ga.defer || ga.next || ga.xmax ||
        ga.norm_w || ga.am_scratch || !ga.xd.dig8 || !fast_ok(w))
        return false;
    if (ga.w2 && (ga.w2->fmt != w->fmt || ga.w2->in_dim != w->in_dim ||
                  ga.w2->row_bytes != w->row_bytes || !fast_ok(ga.w2)))
        return false;
    const int64_t K = w->in_dim;
    return K % 1024 == 0 && K / 1024 <= kRowSplitMaxSteps && ((uintptr_t)ga.xd.dig8 & 15) == 0;
}

int32_t launch_gemv_rowsplit(ut_ctx *ctx, const GemvArgs &ga) {
    if (!gemv_rowsplit_ok(ga)) {
        set_error(ctx, "gemv_rowsplit: one or two rows of an int8 weight with K %% 1024 == 0, "
                       "K <= 8192");
        return UT_ERR_ARG;
    }
    const ut_qtensor *w = ga.w, *w2 = ga.w2;
    PlainArgs a{};
    a.w = (const uint8_t *)w->payload;
    a.scales = w->scales;
    a.O1 = w->out_dim;
    a.w2 = w2 ? (const uint8_t *)w2->payload : a.w;
    a.scales2 = w2 ? w2->scales : a.scales;
    a.O = w->out_dim + (w2 ? w2->out_dim : 0);
    a.K = w->in_dim;
    a.row_bytes = w->row_bytes;
    a.out = ga.out;
    a.ldo = ga.ldo;
    a.out2 = w2 ? ga.out2 : a.out;
    a.ldo2 = w2 ? ga.ldo2 : a.ldo;
    a.accumulate = ga.accumulate;
    a.x.dig = ga.xd.dig8;
    a.x.KW = (w->in_dim + 3) / 4;
    a.exps = ga.xd.exps;
    a.ks = 1;
    int tok = timing_begin(ctx, "gemv_int8_rowsplit");
    const dim3 grid((unsigned)((a.O + 3) / 4));
    if (ga.M == 1)
        hipLaunchKernelGGL(k_gemv_i8_rowsplit<1>, grid, dim3(kGemvThreads), 0, ctx->stream, a);
    else
        hipLaunchKernelGGL(k_gemv_i8_rowsplit<2>, grid, dim3(kGemvThreads), 0, ctx->stream, a);
    timing_end(ctx, tok);
    return launch_check(ctx, "k_gemv_i8_rowsplit");
}

// The value of (m, row) from split-K partials [ks][M][O]: summed in z order
// (integers exactly, f32 in that fixed order) with the row epilogue.
template <int FMT>
__device__ __forceinline__ float splitk_value(const int64_t *__restrict__ part, int ks, int64_t O,
                                              int M, int64_t m, int64_t row, int32_t exp,
                                              float scale) {
    const int64_t zs = (int64_t)M * O, i = m * O + row;
    if constexpr (FMT == UT_FMT_F32) {
        float v = __uint_as_float((uint32_t)part[i]);
#pragma unroll 16
        for (int z = 1; z < ks; z++) v = __fadd_rn(v, __uint_as_float((uint32_t)part[z * zs + i]));
        return v;
    } else {
        int64_t S = part[i];
#pragma unroll 16
        for (int z = 1; z < ks; z++) S += part[z * zs + i];
        return int_total_to_f32(S, exp, scale);
    }
}

template <int FMT>
__global__ __launch_bounds__(256) void k_gemv_splitk_sum(PlainArgs a, int M) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= a.O * M) return;
    const int64_t m = i / a.O, row = i - m * a.O;
    const float v = splitk_value<FMT>(a.part, a.ks, a.O, M, m, row,
                                      FMT == UT_FMT_F32 ? 0 : a.exps[m],
                                      FMT == UT_FMT_F32 ? 0.0f : plain_scale(a, row));
    float *o = plain_out(a, m, row);
    *o = a.accumulate ? __fadd_rn(*o, v) : v;
}

// k_gemv_splitk_sum with argmax partials: grid (ceil(O / 256), M), so each
// workgroup finishes 256 output rows of one activation row and leaves their
// best candidate at a.am[m][blockIdx.x].
template <int FMT>
__global__ __launch_bounds__(256) void k_gemv_splitk_sum_am(PlainArgs a, int M) {
    const int64_t m = blockIdx.y, row = (int64_t)blockIdx.x * 256 + threadIdx.x;
    Best bm[1] = {Best{0.0f, -1}};
    if (row < a.O) {
        const float v = splitk_value<FMT>(a.part, a.ks, a.O, M, m, row,
                                          FMT == UT_FMT_F32 ? 0 : a.exps[m],
                                          FMT == UT_FMT_F32 ? 0.0f : plain_scale(a, row));
        float *o = plain_out(a, m, row);
        const float nv = a.accumulate ? __fadd_rn(*o, v) : v;
        *o = nv;
        argmax_offer(bm[0], nv, row);
    }
    ArgmaxParts p = a.am;
    p.v += m * p.stride;
    p.i += m * p.stride;
    argmax_parts_store<1>(p, bm, blockIdx.x);
}

// The split-K sum for one row per workgroup (thread t: rows 8t..8t+7 of the
// output, each finished exactly as k_gemv_splitk_sum does), then the
// finished row rms-normalised and digitised by the row digitiser's body
// (nd: K = O).  Integer formats, one weight (O1 == O), O % 8 == 0.
template <int FMT>
__global__ __launch_bounds__(1024) void k_splitk_sum_norm(PlainArgs a, int M, RowDigArgs nd) {
    __shared__ double redd[16];
    __shared__ uint32_t redu[16];
    const int m = blockIdx.x, tid = threadIdx.x;
    const int64_t c0 = 8 * (int64_t)tid;
    float v[1][8], wv[1][8];
    if (c0 < a.O) {
        const int64_t zs = (int64_t)M * a.O;
        const int64_t *p = a.part + m * a.O + c0;
        int64_t S[8];
#pragma unroll
        for (int j = 0; j < 8; j++) S[j] = p[j];
#pragma unroll 4
        for (int z = 1; z < a.ks; z++)
#pragma unroll
            for (int j = 0; j < 8; j++) S[j] += p[z * zs + j];
        float *po = a.out + m * a.ldo + c0;
        const float4 s0 = *(const float4 *)(a.scales + c0), s1 = *(const float4 *)(a.scales + c0 + 4);
        const float sc[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
        const float4 w0 = *(const float4 *)(nd.norm_w + c0), w1 = *(const float4 *)(nd.norm_w + c0 + 4);
        float old[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (a.accumulate) {
            const float4 o0 = *(const float4 *)po, o1 = *(const float4 *)(po + 4);
            old[0] = o0.x; old[1] = o0.y; old[2] = o0.z; old[3] = o0.w;
            old[4] = o1.x; old[5] = o1.y; old[6] = o1.z; old[7] = o1.w;
        }
        const int32_t e = a.exps[m];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float x = int_total_to_f32(S[j], e, sc[j]);
            v[0][j] = a.accumulate ? __fadd_rn(old[j], x) : x;
        }
        wv[0][0] = w0.x; wv[0][1] = w0.y; wv[0][2] = w0.z; wv[0][3] = w0.w;
        wv[0][4] = w1.x; wv[0][5] = w1.y; wv[0][6] = w1.z; wv[0][7] = w1.w;
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++) v[0][j] = 0.0f, wv[0][j] = 0.0f;
    }
    // the finished row goes to out after the reductions (nd.raw)
    rowdig_body<1, true>(nd, m, v, wv, redd, redu);
}

// ------------------------------------------------------ generic GEMV ---
// One wave per output row; any K and alignment.  Integer formats sum
// x~ * q exactly (so the result equals the fast kernel's bit for bit);
// f32 sums in a fixed lane order.
__global__ __launch_bounds__(64) void k_gemv_generic(int32_t fmt, const uint8_t *__restrict__ w,
                                                     const float *__restrict__ scales, int64_t O,
                                                     int64_t K, int64_t row_bytes,
                                                     const int32_t *__restrict__ xt,
                                                     const int32_t *__restrict__ exps,
                                                     const float *__restrict__ xf, int64_t ldx,
                                                     int64_t M, float *__restrict__ out,
                                                     int64_t ldo, int accumulate) {
    const int64_t row = blockIdx.x;
    const int lane = threadIdx.x;
    const uint8_t *wr = w + row * row_bytes;
    for (int64_t m = 0; m < M; m++) {
        float v;
        if (fmt == UT_FMT_F32) {
            float acc = 0.0f;
            for (int64_t k = lane; k < K; k += 64)
                acc = __builtin_fmaf(((const float *)wr)[k], xf[m * ldx + k], acc);
            for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
            v = __shfl(acc, 0, 64);
        } else {
            int64_t S = 0;
            for (int64_t k = lane; k < K; k += 64) {
                int q;
                if (fmt == UT_FMT_INT8) q = (int8_t)wr[k];
                else {
                    uint8_t b = wr[k >> 1];
                    int nib = (k & 1) ? (b >> 4) : (b & 0xF);
                    q = (nib ^ 8) - 8;
                }
                S += (int64_t)xt[m * K + k] * q;
            }
            for (int off = 32; off >= 1; off >>= 1) {
                int lo = __shfl_xor((int)(uint32_t)(uint64_t)S, off, 64);
                int hi = __shfl_xor((int)(uint32_t)((uint64_t)S >> 32), off, 64);
                S += (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint64_t)(uint32_t)lo);
            }
            v = int_total_to_f32(S, exps[m], scales[row]);
        }
        if (lane == 0) {
            float *o = out + m * ldo + row;
            *o = accumulate ? __fadd_rn(*o, v) : v;
        }
    }
}

static bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

bool gemv_norm_ok(const ut_qtensor *w, int64_t M, const void *x, const void *norm_w) {
    if (M < 1 || M > 2 || !w || (w->fmt != UT_FMT_INT8 && w->fmt != UT_FMT_INT4))
        return false;
    const int64_t K = w->in_dim;
    const int64_t kc = w->fmt == UT_FMT_INT8 ? gemv_chunk_cols<UT_FMT_INT8, 1, kGemvNormCols>()
                                             : gemv_chunk_cols<UT_FMT_INT4, 1, kGemvNormCols>();
    const int64_t step = w->fmt == UT_FMT_INT8 ? FmtTraits<UT_FMT_INT8>::kStepCols
                                               : FmtTraits<UT_FMT_INT4>::kStepCols;
    return K <= kc && K % step == 0 && K % 4 == 0 && aligned16(x) && aligned16(norm_w) &&
           aligned16(w->payload) && w->row_bytes % 16 == 0;
}

// Whether the fast kernel takes this weight (16-byte aligned rows).
static bool fast_ok(const ut_qtensor *w);
bool gemv_fast_ok(const ut_qtensor *w) { return fast_ok(w); }

static bool fast_ok(const ut_qtensor *w) {
    if (!aligned16(w->payload)) return false;
    if (w->fmt == UT_FMT_INT4) return w->in_dim % 32 == 0;
    if (w->fmt == UT_FMT_INT8) return w->in_dim % 16 == 0;
    return w->in_dim % 4 == 0;
}

// Split of K for a weight of O rows and K columns.  Weights with fewer
// than 256 row tiles cannot keep the chip's loads in flight, so their K
// range is split over blockIdx.z (each split at least two steps wide) and a
// second launch sums the partials.  f32 splits depend on the weight's shape
// only (64-row tiles, about kSplitTargetWGs workgroups), so an f32 row's
// summation order is the same for every M; integer partials are exact, so
// their split follows the launch's own tiles and occupancy.
constexpr int64_t kSplitTargetWGs = 1024;
constexpr int64_t kSplitMinTiles = 256;  // integer formats: at least this many tiles -> no split

// resident: workgroups of the launch's kernel the chip holds at once.
static void splitk_plan(int32_t fmt, int64_t O, int64_t K, int rows_per_wg, int64_t resident,
                        int *ks_out, int64_t *kslice_out) {
    const int64_t step = fmt == UT_FMT_INT4 ? FmtTraits<UT_FMT_INT4>::kStepCols
                         : fmt == UT_FMT_INT8 ? FmtTraits<UT_FMT_INT8>::kStepCols
                                              : FmtTraits<UT_FMT_F32>::kStepCols;
    int64_t ks;
    if (fmt == UT_FMT_F32) {
        // f32 partials are summed in z order, so their split must not depend
        // on the row count: 64-row tiles, about kSplitTargetWGs workgroups
        const int64_t tiles64 = (O + 63) / 64;
        ks = tiles64 >= 256 ? 1 : (kSplitTargetWGs + tiles64 - 1) / tiles64;
    } else {
        // integer partials are exact, so the launch's own tiles decide: as
        // many splits as fit the chip in one wave of workgroups (a second,
        // partial wave would only add a tail)
        const int64_t tiles = (O + rows_per_wg - 1) / rows_per_wg;
        ks = tiles >= kSplitMinTiles ? 1 : resident / tiles;
        if (ks < 1) ks = 1;
    }
    const int64_t max_ks = K / (2 * step);
    if (ks > max_ks) ks = max_ks;
    // partials of the widest case (M = 4) must fit
    while (ks > 1 && ks * 4 * O * 8 > kSplitKPartBytes) ks--;
    if (ks <= 1) {
        *ks_out = 1;
        *kslice_out = K;
        return;
    }
    int64_t kslice = (K + ks - 1) / ks;
    kslice = (kslice + step - 1) / step * step;
    *ks_out = (int)((K + kslice - 1) / kslice);
    *kslice_out = kslice;
}

// Workgroups of k_gemv<FMT, M> resident on the whole chip (occupancy query,
// once per instantiation).
template <int FMT, int M> static int64_t gemv_resident_m(ut_ctx *ctx) {
    // sessions on several threads may ask at once: the same answer either way
    static std::atomic<int> per_cu{0};
    int n = per_cu.load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, (const void *)k_gemv<FMT, M>,
                                                         kGemvThreads, 0) != hipSuccess ||
            n < 1) {
            (void)hipGetLastError();
            n = 2;
        }
        per_cu.store(n, std::memory_order_relaxed);
    }
    return (int64_t)n * ctx->multiprocessors;
}
template <int FMT> static int64_t gemv_resident(ut_ctx *ctx, int mrows) {
    switch (mrows) {
    case 1: return gemv_resident_m<FMT, 1>(ctx);
    case 2: return gemv_resident_m<FMT, 2>(ctx);
    case 3: return gemv_resident_m<FMT, 3>(ctx);
    default: return gemv_resident_m<FMT, 4>(ctx);
    }
}

// After a split-K GEMV launch: the consumer sums the partials (defer), or
// the sum runs fused with the next rmsnorm + digitise, or alone.
template <int FMT>
static int32_t splitk_finish(ut_ctx *ctx, const GemvArgs &ga, const PlainArgs &a, int64_t m0,
                             int mrows, const char *name) {
    UT_TRY(launch_check(ctx, name));
    const ut_qtensor *w2 = ga.w2;
    const bool fuse_next = FMT != UT_FMT_F32 && ga.next && !ga.defer && !w2 && m0 == 0 &&
                           mrows == ga.M && a.O % 8 == 0 && a.O <= 8 * 1024 &&
                           aligned16(a.out) && a.ldo % 4 == 0 && aligned16(a.scales) &&
                           aligned16(ga.next->norm_w) && ga.next->nd.exps;
    if (ga.defer) {
        // the consumer sums the partials (only one chunk of rows)
        ga.defer->part = a.part;
        ga.defer->ks = a.ks;
        ga.defer->O = a.O;
    } else if (fuse_next) {
        const NormNext &nx = *ga.next;
        RowDigArgs nd{};
        nd.K = a.O;
        nd.norm_w = nx.norm_w;
        nd.eps = nx.eps;
        nd.out = nx.normed;
        nd.ldo = nx.ldn;
        nd.exps = nx.nd.exps;
        nd.dig4 = (nx.flags & XD_DIG4) ? nx.nd.dig4 : nullptr;
        nd.dig8 = (nx.flags & XD_DIG8) ? nx.nd.dig8 : nullptr;
        nd.xt = (nx.flags & XD_XT) ? nx.nd.xt : nullptr;
        nd.raw = a.out;
        nd.raw2 = nx.raw2;
        nd.ldr2 = nx.ld2;
        nd.pos2 = nx.pos2;
        nd.ldr = a.ldo;
        const unsigned threads = (unsigned)((a.O / 8 + 63) / 64 * 64);
        hipLaunchKernelGGL(k_splitk_sum_norm<FMT>, dim3((unsigned)mrows), dim3(threads), 0,
                           ctx->stream, a, mrows, nd);
        if (ga.next_done) *ga.next_done = true;
    } else if (a.am.v) {
        // argmax partials per 256 finished rows (a.am's stride was set so)
        hipLaunchKernelGGL(k_gemv_splitk_sum_am<FMT>, dim3((unsigned)((a.O + 255) / 256), (unsigned)mrows),
                           dim3(256), 0, ctx->stream, a, mrows);
    } else {
        const int64_t n = a.O * mrows;
        hipLaunchKernelGGL(k_gemv_splitk_sum<FMT>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                           ctx->stream, a, mrows);
    }
    return UT_OK;
}

// The argmax partials' view for a launch of gx workgroups of rows_per_wg
// output rows (ks > 1: the split sum's 256-row workgroups), when the caller
// asked for them (ga.am_scratch) and the launch finishes every row of the
// call: one chunk of rows, one weight, no deferred or fused consumer.
static void argmax_plan(const GemvArgs &ga, PlainArgs &a, int64_t m0, int mrows, int64_t gx) {
    a.am = ArgmaxParts{};
    if (!ga.am_scratch || !ga.am_out || ga.w2 || ga.defer || ga.next || m0 != 0 || mrows != ga.M)
        return;
    const int64_t stride = a.ks > 1 ? (a.O + 255) / 256 : gx;
    if (stride > argmax_gemv_parts_max(a.O)) return;
    a.am = argmax_parts_view(ga.am_scratch, mrows, stride);
    *ga.am_out = a.am;
}

// Workgroups of k_gemv_mfma_i8<M, F32X> resident on the chip.
template <int M, bool F32X> static int64_t gemv_i8_mfma_resident(ut_ctx *ctx) {
    static std::atomic<int> per_cu{0};
    int n = per_cu.load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, (const void *)k_gemv_mfma_i8<M, F32X>,
                                                         kGemvThreads, 0) != hipSuccess ||
            n < 1) {
            (void)hipGetLastError();
            n = 2;
        }
        per_cu.store(n, std::memory_order_relaxed);
    }
    return (int64_t)n * ctx->multiprocessors;
}

// Weights of at least this many rows (the LM head) take two 16-row tiles
// per wave: half the activation staging per weight byte (config-4 four-row
// LM head 166.8 -> 161.3 us); the other launches keep one (fewer, fatter
// workgroups measured slower there).
constexpr int64_t kI8MfmaWideRows = 65536;

template <int M, bool F32X, int TW = gemv_i8_mfma_tw<M>()>
static int32_t launch_i8_mfma_m(ut_ctx *ctx, const GemvArgs &ga, PlainArgs a, int64_t m0) {
    if constexpr (!F32X && TW == 1) {
        if (a.O >= kI8MfmaWideRows) return launch_i8_mfma_m<M, F32X, 2>(ctx, ga, a, m0);
    }
    constexpr int rows_per_wg = 64 * TW;
    // a launch that reduces the producer's partial maxima pays that in every
    // workgroup: half as many splits, as for k_gemv
    const int64_t resident = gemv_i8_mfma_resident<M, F32X>(ctx) / (F32X ? 2 : 1);
    splitk_plan(UT_FMT_INT8, a.O, a.K, rows_per_wg, resident, &a.ks, &a.kslice);
#if UT_GEMV_I8_MFMA_SPLIT_FILL
    {
        // split until the launch fills the chip's resident workgroups once
        const int64_t tiles = (a.O + rows_per_wg - 1) / rows_per_wg;
        int64_t ks = resident / tiles;
        const int64_t step = kMfmaI8SegCols;
        if (ks > a.K / (2 * step)) ks = a.K / (2 * step);
        while (ks > 1 && ks * 4 * a.O * 8 > kSplitKPartBytes) ks--;
        if (ks > a.ks) {
            a.kslice = ((a.K + ks - 1) / ks + step - 1) / step * step;
            a.ks = (int)((a.K + a.kslice - 1) / a.kslice);
        }
    }
#endif
    a.part = nullptr;
    if (a.ks > 1) UT_TRY(splitk_buffer(ctx, &a.part));
    const dim3 grid((unsigned)((a.O + rows_per_wg - 1) / rows_per_wg), 1, (unsigned)a.ks);
    argmax_plan(ga, a, m0, M, grid.x);
    const char *name = "gemv_int8_mfma";
    int tok = timing_begin(ctx, name);
    hipLaunchKernelGGL((k_gemv_mfma_i8<M, F32X, TW>), grid, dim3(kGemvThreads), 0, ctx->stream, a);
    if (a.ks > 1) UT_TRY(splitk_finish<UT_FMT_INT8>(ctx, ga, a, m0, M, name));
    timing_end(ctx, tok);
    return launch_check(ctx, name);
}

static int32_t launch_gemv_i8_mfma(ut_ctx *ctx, const GemvArgs &ga, const PlainArgs &a, int64_t m0,
                                   int mrows) {
    const bool f32x = a.xmax != nullptr;
    switch (mrows) {
    case 3: return f32x ? launch_i8_mfma_m<3, true>(ctx, ga, a, m0) : launch_i8_mfma_m<3, false>(ctx, ga, a, m0);
    case 4: return f32x ? launch_i8_mfma_m<4, true>(ctx, ga, a, m0) : launch_i8_mfma_m<4, false>(ctx, ga, a, m0);
#if UT_GEMV_I8_MFMA_MIN_M <= 2
    case 2: return f32x ? launch_i8_mfma_m<2, true>(ctx, ga, a, m0) : launch_i8_mfma_m<2, false>(ctx, ga, a, m0);
#endif
    default: return UT_ERR_ARG;
    }
}

template <int FMT>
static int32_t launch_fast(ut_ctx *ctx, const GemvArgs &ga, int64_t m0, int mrows) {
    const ut_qtensor *w = ga.w, *w2 = ga.w2;
    PlainArgs a;
    a.w = (const uint8_t *)w->payload;
    a.scales = w->scales;
    a.O1 = w->out_dim;
    a.w2 = w2 ? (const uint8_t *)w2->payload : a.w;
    a.scales2 = w2 ? w2->scales : a.scales;
    a.O = w->out_dim + (w2 ? w2->out_dim : 0);
    a.K = w->in_dim;
    a.row_bytes = w->row_bytes;
    a.out = ga.out + m0 * ga.ldo;
    a.ldo = ga.ldo;
    a.out2 = w2 ? ga.out2 + m0 * ga.ldo2 : a.out;
    a.ldo2 = w2 ? ga.ldo2 : a.ldo;
    a.accumulate = ga.accumulate;
    if constexpr (FMT == UT_FMT_F32) {
        a.x.xf = ga.xf + m0 * w->in_dim;
        a.x.ldx = w->in_dim;
        a.x.dig = nullptr;
        a.x.KW = 0;
        a.exps = nullptr;
        if (!aligned16(a.x.xf)) return UT_ERR_ARG;
    } else {
        constexpr int PL = FmtTraits<FMT>::kPlanes;
        const int64_t KW = (w->in_dim + FmtTraits<FMT>::kColsPerWord - 1) / FmtTraits<FMT>::kColsPerWord;
        if (ga.norm_w) {
            // one or two rows, normalised and digitised while staged (gemv
            // checked the shape: one chunk, no split)
            a.x.dig = nullptr;
            a.x.KW = KW;
            a.x.xf = ga.xf;
            a.x.ldx = w->in_dim;
            a.x.nw = ga.norm_w;
            a.x.neps = ga.norm_eps;
            a.exps = nullptr;
        } else if (ga.xmax) {
            a.x.dig = nullptr;
            a.x.KW = KW;
            a.x.xf = ga.xf + m0 * w->in_dim;
            a.x.ldx = w->in_dim;
            a.exps = ga.exps_out + m0;
            if (!aligned16(a.x.xf)) return UT_ERR_ARG;
        } else {
            a.x.dig = (FMT == UT_FMT_INT4 ? ga.xd.dig4 : ga.xd.dig8) + m0 * PL * KW;
            a.x.KW = KW;
            a.x.xf = nullptr;
            a.x.ldx = 0;
            a.exps = ga.xd.exps + m0;
        }
    }
    a.xmax = FMT != UT_FMT_F32 && ga.xmax ? ga.xmax + m0 * ga.nxmax : nullptr;
    a.nxmax = ga.nxmax;
    // int8 at 3..4 rows: the matrix-core kernel (64-row tiles, steps of 64
    // columns), the same partials and epilogue
    const bool i8_mfma = FMT == UT_FMT_INT8 && !ga.norm_w && mrows >= UT_GEMV_I8_MFMA_MIN_M && mrows <= 4 &&
                         w->in_dim % kMfmaI8SegCols == 0 &&
                         (a.xmax || ((uintptr_t)a.x.dig & 15) == 0);
    if (i8_mfma) return launch_gemv_i8_mfma(ctx, ga, a, m0, mrows);
    const int rows_per_wg = plain_rows_rt(mrows);
    // a launch that reduces the producer's partial maxima while staging
    // pays that in every workgroup: half as many splits (o_proj at
    // DeepSeek-V3 width: 2 splits against 4 took the GEMV from 27.0 to
    // 25.3 us and its split sum from 12.0 to 10.2 us)
    const int64_t resident = gemv_resident<FMT>(ctx, mrows) / (a.xmax ? 2 : 1);
    splitk_plan(FMT, a.O, w->in_dim, rows_per_wg, resident, &a.ks, &a.kslice);
    if (ga.norm_w) {
        // the staging normalises whole rows: no K split
        a.ks = 1;
        a.kslice = w->in_dim;
    } else if (FMT != UT_FMT_F32) {
        // every launch takes enough splits for its K slice to be staged in
        // one chunk at its row count: a second chunk drains the weight stream
        // behind a staging round (o_proj at DeepSeek-V3 width, two rows: 2
        // splits of 8,192 columns against 4 of 4,096 took the GEMV from 37.3
        // to 26.7 us for 1.9 us more in its split sum; at four rows the
        // occupancy rule alone left it unsplit, eight 2,048-column chunks)
        const int64_t kc = mrows == 1   ? gemv_chunk_cols<FMT, 1>()
                           : mrows == 2 ? gemv_chunk_cols<FMT, 2>()
                           : mrows == 3 ? gemv_chunk_cols<FMT, 3>()
                                        : gemv_chunk_cols<FMT, 4>();
        if (a.kslice > kc) {
            constexpr int64_t step = FmtTraits<FMT>::kStepCols;
            const int64_t K = w->in_dim;
            int64_t ks = (K + kc - 1) / kc;
            while (ks > 1 && ks * 4 * a.O * 8 > kSplitKPartBytes) ks--;  // as splitk_plan
            a.kslice = ((K + ks - 1) / ks + step - 1) / step * step;
            a.ks = (int)((K + a.kslice - 1) / a.kslice);
        }
    }
    a.part = nullptr;
    if (a.ks > 1) UT_TRY(splitk_buffer(ctx, &a.part));
    dim3 grid((unsigned)((a.O + rows_per_wg - 1) / rows_per_wg), 1, (unsigned)a.ks);
    argmax_plan(ga, a, m0, mrows, grid.x);
    const char *name = FMT == UT_FMT_INT4 ? "gemv_int4" : FMT == UT_FMT_INT8 ? "gemv_int8" : "gemv_f32";
    int tok = timing_begin(ctx, name);
    if constexpr (FMT != UT_FMT_F32) {
        if (ga.norm_w) {
            if (ga.kv) {
                a.kv = *ga.kv;
                grid.x += (unsigned)mrows;  // the kv appends' workgroups
            }
            if (mrows == 1)
                hipLaunchKernelGGL((k_gemv<FMT, 1, true>), grid, dim3(kGemvThreads), 0, ctx->stream, a);
            else
                hipLaunchKernelGGL((k_gemv<FMT, 2, true>), grid, dim3(kGemvThreads), 0, ctx->stream, a);
            timing_end(ctx, tok);
            return launch_check(ctx, name);
        }
    }
    switch (mrows) {
    case 1: hipLaunchKernelGGL((k_gemv<FMT, 1>), grid, dim3(kGemvThreads), 0, ctx->stream, a); break;
    case 2: hipLaunchKernelGGL((k_gemv<FMT, 2>), grid, dim3(kGemvThreads), 0, ctx->stream, a); break;
    case 3: hipLaunchKernelGGL((k_gemv<FMT, 3>), grid, dim3(kGemvThreads), 0, ctx->stream, a); break;
    default: hipLaunchKernelGGL((k_gemv<FMT, 4>), grid, dim3(kGemvThreads), 0, ctx->stream, a); break;
    }
    if (a.ks > 1) UT_TRY(splitk_finish<FMT>(ctx, ga, a, m0, mrows, name));
    timing_end(ctx, tok);
    return launch_check(ctx, name);
}

// f32 weights with few output rows (the router gate: 256 x 7168): one
// workgroup per output row for all M <= 4 activation rows; thread t takes
// the float4 columns 4t + 1024j (x's columns and the row's weights loaded
// first, every load in flight at once; NJ exact for the row where it can
// be: config-4 router at four rows 10.3 -> 5.4 us), the per-thread FMA
// chains are summed by DPP within each wave and then over the four waves in
// order.  EPW (output rows per workgroup, reusing x's registers) stays 1:
// four rows per workgroup at four activation rows measured 7.0 us.  No
// split-K partials, so the router reads the logits directly.
template <int M, int NJ, int EPW>
__global__ __launch_bounds__(256) void k_rowdot_f32(const float *__restrict__ w, int64_t K,
                                                    const float *__restrict__ x, int64_t ldx,
                                                    float *__restrict__ out, int64_t ldo,
                                                    int64_t O) {
    __shared__ float red[EPW][4][M];
    const int tid = threadIdx.x;
    float4 xv[M][NJ];
#pragma unroll
    for (int m = 0; m < M; m++)
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int64_t c = 4 * tid + 1024 * j;
            xv[m][j] = c < K ? ld_global<float4>(x + m * ldx + c) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    float4 wv[EPW][NJ];
#pragma unroll
    for (int e = 0; e < EPW; e++) {
        const int64_t row0 = (int64_t)blockIdx.x * EPW + e;
        const float *wr = w + (row0 < O ? row0 : O - 1) * K;
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int64_t c = 4 * tid + 1024 * j;
            wv[e][j] = c < K ? ld_global<float4>(wr + c) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    }
#pragma unroll
    for (int e = 0; e < EPW; e++)
#pragma unroll
        for (int m = 0; m < M; m++) {
            float a = 0.0f;
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                const int64_t c = 4 * tid + 1024 * j;
                if (c < K) {
                    a = __builtin_fmaf(wv[e][j].x, xv[m][j].x, a);
                    a = __builtin_fmaf(wv[e][j].y, xv[m][j].y, a);
                    a = __builtin_fmaf(wv[e][j].z, xv[m][j].z, a);
                    a = __builtin_fmaf(wv[e][j].w, xv[m][j].w, a);
                }
            }
            a = wave_reduce_dpp(a, [](float p, float q) { return p + q; });
            if ((tid & 63) == 0) red[e][tid >> 6][m] = a;
        }
    __syncthreads();
    if (tid < EPW * M) {
        const int e = tid / M, m = tid - e * M;
        const int64_t row = (int64_t)blockIdx.x * EPW + e;
        if (row < O) out[m * ldo + row] = ((red[e][0][m] + red[e][1][m]) + red[e][2][m]) + red[e][3][m];
    }
}

bool rowdot_f32_ok(const ut_qtensor *w, int64_t M) {
    return w->fmt == UT_FMT_F32 && M >= 1 && M <= 4 && w->in_dim % 4 == 0 &&
           w->in_dim <= 8 * 1024 && w->out_dim <= 4096 && ((uintptr_t)w->payload & 15) == 0;
}

int32_t launch_rowdot_f32(ut_ctx *ctx, const ut_qtensor *w, const float *x, int64_t M,
                          float *out, int64_t ldo) {
    if (!rowdot_f32_ok(w, M) || ((uintptr_t)x & 15) != 0) {
        set_error(ctx, "rowdot_f32: unsupported shape or alignment");
        return UT_ERR_ARG;
    }
    const int64_t K = w->in_dim, O = w->out_dim;
    const int nj = (int)((K + 1023) / 1024);
    int tok = timing_begin(ctx, "rowdot_f32");
    const float *wp = (const float *)w->payload;
#define UT_RD(MM, NJ, EPW)                                                                  \
    hipLaunchKernelGGL((k_rowdot_f32<MM, NJ, EPW>), dim3((unsigned)((O + EPW - 1) / EPW)), \
                       dim3(256), 0, ctx->stream, wp, K, x, K, out, ldo, O)
#define UT_RDM(MM, EPW)                                              \
    do {                                                             \
        if (nj <= 2) UT_RD(MM, 2, EPW);                              \
        else if (nj <= 4) UT_RD(MM, 4, EPW);                         \
        else if (nj == 7) UT_RD(MM, 7, EPW);                         \
        else UT_RD(MM, 8, EPW);                                      \
    } while (0)
    switch (M) {
    case 1: UT_RDM(1, 1); break;
    case 2: UT_RDM(2, 1); break;
    case 3: UT_RDM(3, 1); break;
    default: UT_RDM(4, 1); break;
    }
#undef UT_RDM
#undef UT_RD
    timing_end(ctx, tok);
    return launch_check(ctx, "k_rowdot_f32");
}

int32_t gemv(ut_ctx *ctx, const GemvArgs &ga) {
    const ut_qtensor *w = ga.w;
    if (ga.defer) ga.defer->ks = 1;
    if (ga.am_out) *ga.am_out = ArgmaxParts{};
    if (ga.next_done) *ga.next_done = false;
    if (ga.M <= 0) return UT_OK;
    if (ga.w2 && (ga.w2->fmt != w->fmt || ga.w2->in_dim != w->in_dim ||
                  ga.w2->row_bytes != w->row_bytes || !fast_ok(ga.w2) || !fast_ok(w) ||
                  (w->fmt == UT_FMT_F32 && !aligned16(ga.xf)))) {
        set_error(ctx, "gemv: the two weights must share format, K and row layout");
        return UT_ERR_ARG;
    }
    if (ga.defer && ga.M > 4) {
        set_error(ctx, "gemv: deferred split-K sums take at most 4 rows");
        return UT_ERR_ARG;
    }
    if (ga.norm_w && (ga.w2 || ga.defer || ga.next || ga.xmax || !gemv_norm_ok(w, ga.M, ga.xf, ga.norm_w))) {
        set_error(ctx, "gemv: normalise-while-staging takes one or two rows of at most 2048 "
                       "columns (a multiple of the step) of an int4/int8 weight, 16-byte aligned");
        return UT_ERR_ARG;
    }
    if (fast_ok(w) && (w->fmt == UT_FMT_F32 ? aligned16(ga.xf) && (w->in_dim % 4 == 0) : true)) {
        for (int64_t m0 = 0; m0 < ga.M; m0 += 4) {
            int mrows = (int)((ga.M - m0) < 4 ? (ga.M - m0) : 4);
            int32_t rc;
            if (w->fmt == UT_FMT_INT4) rc = launch_fast<UT_FMT_INT4>(ctx, ga, m0, mrows);
            else if (w->fmt == UT_FMT_INT8) rc = launch_fast<UT_FMT_INT8>(ctx, ga, m0, mrows);
            else rc = launch_fast<UT_FMT_F32>(ctx, ga, m0, mrows);
            if (rc) return rc;
        }
        return UT_OK;
    }
    if (w->fmt != UT_FMT_F32 && !ga.xd.xt) {
        set_error(ctx, "generic GEMV needs x~ (XD_XT) digits");
        return UT_ERR_ARG;
    }
    int tok = timing_begin(ctx, "gemv_generic");
    hipLaunchKernelGGL(k_gemv_generic, dim3((unsigned)w->out_dim), dim3(64), 0, ctx->stream, w->fmt,
                       (const uint8_t *)w->payload, w->scales, w->out_dim, w->in_dim, w->row_bytes,
                       ga.xd.xt, ga.xd.exps, ga.xf, w->in_dim, ga.M, ga.out, ga.ldo, ga.accumulate);
    timing_end(ctx, tok);
    return launch_check(ctx, "k_gemv_generic");
}

size_t matmul_digit_bytes(int64_t M, int64_t K) {
    return xdigits_bytes(M, K, XD_DIG4 | XD_DIG8 | XD_XT);
}

// ------------------------------------------------------ fast int8 ---
// The opt-in fast-int8 path (undertow-quant/src/lib.rs:31-59,
// avx512.rs:221-242).  k_act_quant_i8: one workgroup per activation row,
// quantize_activations: max = max|v| over the row skipping NaN (f32::max
// keeps the non-NaN operand, fmaxf too), scale = max/127, inv = 127/max,
// code = round(v*inv) half away from zero, clamped to +-127, NaN -> 0; a
// zero row gets scale 0 and zero codes.  Rows of xq are kp bytes (zero
// padded to 16).
__global__ __launch_bounds__(256) void k_act_quant_i8(const float *__restrict__ x, int64_t K,
                                                      int8_t *__restrict__ xq, int64_t kp,
                                                      float *__restrict__ ascale) {
    __shared__ float red[4];
    const int64_t m = blockIdx.x;
    const float *xr = x + m * K;
    float mx = 0.0f;
    for (int64_t i = threadIdx.x; i < K; i += 256) mx = fmaxf(mx, fabsf(xr[i]));
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const bool zero = mx == 0.0f;
    const float inv = zero ? 0.0f : __fdiv_rn(127.0f, mx);
    if (threadIdx.x == 0) ascale[m] = zero ? 0.0f : __fdiv_rn(mx, 127.0f);
    int8_t *qr = xq + m * kp;
    for (int64_t i = threadIdx.x; i < kp; i += 256) {
        int q = 0;
        if (i < K && !zero) {
            const float t = roundf(__fmul_rn(xr[i], inv));
            q = isnan(t) ? 0 : (int)fminf(fmaxf(t, -127.0f), 127.0f);
        }
        qr[i] = (int8_t)q;
    }
}

// One wave per output row: the exact integer dot of the row's i8 codes and
// the row's quantised activations (v_dot4 over 16-byte steps when K % 16 ==
// 0, bytes otherwise), then (acc as f32) * a_scale * scale[o].  Grid
// (ceil(O / 4), seq).
__global__ __launch_bounds__(256) void k_gemv_fast_i8(const int8_t *__restrict__ w,
                                                      const float *__restrict__ scales, int64_t O,
                                                      int64_t K, const int8_t *__restrict__ xq,
                                                      int64_t kp, const float *__restrict__ ascale,
                                                      float *__restrict__ out, int64_t ldo,
                                                      int accumulate) {
    const int64_t o = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t m = blockIdx.y;
    const int lane = threadIdx.x & 63;
    if (o >= O) return;
    const int8_t *wr = w + o * K;
    const int8_t *xr = xq + m * kp;
    int32_t acc = 0;
    if ((K & 15) == 0) {
        for (int64_t c = 16 * (int64_t)lane; c < K; c += 1024) {
            const uint4 wv = ld_weights(wr + c);
            const uint4 xv = *(const uint4 *)(xr + c);
            acc = __builtin_amdgcn_sdot4((int)wv.x, (int)xv.x, acc, false);
            acc = __builtin_amdgcn_sdot4((int)wv.y, (int)xv.y, acc, false);
            acc = __builtin_amdgcn_sdot4((int)wv.z, (int)xv.z, acc, false);
            acc = __builtin_amdgcn_sdot4((int)wv.w, (int)xv.w, acc, false);
        }
    } else {
        for (int64_t c = lane; c < K; c += 64) acc += (int32_t)wr[c] * (int32_t)xr[c];
    }
    for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (lane == 0) {
        const float v = __fmul_rn(__fmul_rn((float)acc, ascale[m]), scales[o]);
        float *po = out + m * ldo + o;
        *po = accumulate ? __fadd_rn(*po, v) : v;
    }
}

int32_t matmul_fast_i8(ut_ctx *ctx, const ut_qtensor *qt, float *out, int64_t ldo, int accumulate,
                       const float *x, int64_t seq) {
    const int64_t K = qt->in_dim, O = qt->out_dim, kp = (K + 15) / 16 * 16;
    ScratchPlan plan;
    plan.add((size_t)(seq * kp));
    plan.add((size_t)seq * 4);
    std::vector<void *> ptrs;
    UT_TRY(scratch_acquire(ctx, plan, ptrs));
    int8_t *xq = (int8_t *)ptrs[0];
    float *as = (float *)ptrs[1];
    int tok = timing_begin(ctx, "gemv_fast_i8");
    hipLaunchKernelGGL(k_act_quant_i8, dim3((unsigned)seq), dim3(256), 0, ctx->stream, x, K, xq,
                       kp, as);
    hipLaunchKernelGGL(k_gemv_fast_i8, dim3((unsigned)((O + 3) / 4), (unsigned)seq), dim3(256), 0,
                       ctx->stream, (const int8_t *)qt->payload, qt->scales, O, K, xq, kp, as, out,
                       ldo, accumulate);
    timing_end(ctx, tok);
    return launch_check(ctx, "k_gemv_fast_i8");
}


int32_t matmul_digits(ut_ctx *ctx, const ut_qtensor *w, const float *x, const XDigits &xd,
                      int64_t M, float *out, int64_t ldo, int accumulate) {
    // the opt-in fast-int8 path replaces every int8 QTensor::matmul
    // (qtensor.rs:385-398): activations quantised per row from x itself
    if (ctx->fast_int8 && w->fmt == UT_FMT_INT8 && M > 0)
        return matmul_fast_i8(ctx, w, out, ldo, accumulate, x, M);
    GemvArgs ga;
    ga.w = w;
    ga.M = M;
    ga.out = out;
    ga.ldo = ldo;
    ga.accumulate = accumulate;
    ga.xf = x;
    ga.xd = xd;
    if (w->fmt != UT_FMT_F32) {
        const bool need4 = w->fmt == UT_FMT_INT4 && fast_ok(w), need8 = w->fmt == UT_FMT_INT8 && fast_ok(w);
        if ((need4 && !xd.dig4) || (need8 && !xd.dig8) || (!fast_ok(w) && !xd.xt)) {
            set_error(ctx, "matmul_digits: activation digits of the wrong form");
            return UT_ERR_ARG;
        }
    }
    return gemv(ctx, ga);
}

int32_t matmul_digits_argmax(ut_ctx *ctx, const ut_qtensor *w, const float *x, const XDigits &xd,
                             int64_t M, float *out, int32_t *idx, void *am_scratch,
                             const int32_t *err, const int32_t *tail, int ntail) {
    ArgmaxParts am;
    if (!(ctx->fast_int8 && w->fmt == UT_FMT_INT8) && w->fmt != UT_FMT_F32 && fast_ok(w) &&
        M >= 1 && M <= 4) {
        GemvArgs ga;
        ga.w = w;
        ga.M = M;
        ga.out = out;
        ga.ldo = w->out_dim;
        ga.xf = x;
        ga.xd = xd;
        ga.am_scratch = am_scratch;
        ga.am_out = &am;
        const bool need4 = w->fmt == UT_FMT_INT4, need8 = w->fmt == UT_FMT_INT8;
        if ((need4 && !xd.dig4) || (need8 && !xd.dig8)) {
            set_error(ctx, "matmul_digits: activation digits of the wrong form");
            return UT_ERR_ARG;
        }
        UT_TRY(gemv(ctx, ga));
    } else {
        UT_TRY(matmul_digits(ctx, w, x, xd, M, out, w->out_dim, 0));
    }
    if (am.v) return launch_argmax_final(ctx, out, M, w->out_dim, am, idx, err, tail, ntail);
    return launch_argmax(ctx, out, M, w->out_dim, w->out_dim, idx, am_scratch, err, tail, ntail);
}

int32_t matmul_dev(ut_ctx *ctx, const ut_qtensor *w, const float *x, int64_t M, float *out,
                   int64_t ldo, int accumulate, void *digit_scratch) {
    if (M <= 0) return UT_OK;
    if (ctx->fast_int8 && w->fmt == UT_FMT_INT8)
        return matmul_fast_i8(ctx, w, out, ldo, accumulate, x, M);
    GemvArgs ga;
    ga.w = w;
    ga.M = M;
    ga.out = out;
    ga.ldo = ldo;
    ga.accumulate = accumulate;
    if (w->fmt == UT_FMT_F32) {
        ga.xf = x;
        return gemv(ctx, ga);
    }
    int flags = fast_ok(w) ? xdigit_flags_for(w->fmt, w->in_dim) : XD_XT;
    ga.xd = xdigits_view(digit_scratch, M, w->in_dim, flags);
    UT_TRY(launch_digitize(ctx, x, w->in_dim, M, w->in_dim, nullptr, ga.xd, flags));
    return gemv(ctx, ga);
}

}  // namespace ut

using namespace ut;

extern "C" int32_t ut_set_fast_int8(ut_ctx *ctx, int32_t enabled) {
    if (!ctx) return UT_ERR_ARG;
    ctx->fast_int8 = enabled != 0;
    return UT_OK;
}

extern "C" int32_t ut_fast_int8_enabled(const ut_ctx *ctx) { return ctx && ctx->fast_int8 ? 1 : 0; }

extern "C" int32_t ut_qtensor_matmul(ut_ctx *ctx, const ut_qtensor *qt, float *out_dev,
                                     int64_t out_len, const float *x_dev, int64_t x_len,
                                     int64_t seq) {
    if (!ctx || !qt || !out_dev || !x_dev || seq < 0) {
        set_error(ctx, "ut_qtensor_matmul: bad argument");
        return UT_ERR_ARG;
    }
    // the reference's assert_eq!s (qtensor.rs:283-284)
    if (x_len != seq * qt->in_dim) {
        set_error(ctx, "x shape: %lld != %lld*%lld", (long long)x_len, (long long)seq,
                  (long long)qt->in_dim);
        return UT_ERR_SHAPE;
    }
    if (out_len != seq * qt->out_dim) {
        set_error(ctx, "out shape: %lld != %lld*%lld", (long long)out_len, (long long)seq,
                  (long long)qt->out_dim);
        return UT_ERR_SHAPE;
    }
    if (seq == 0) return UT_OK;
    // Int8 { .. } if fast_int8_enabled() (qtensor.rs:385-398)
    if (qt->fmt == UT_FMT_INT8 && ctx->fast_int8)
        return matmul_fast_i8(ctx, qt, out_dev, qt->out_dim, 0, x_dev, seq);
    GemvArgs ga;
    ga.w = qt;
    ga.M = seq;
    ga.out = out_dev;
    ga.ldo = qt->out_dim;
    if (qt->fmt == UT_FMT_F32) {
        ga.xf = x_dev;
        return gemv(ctx, ga);
    }
    int flags = xdigit_flags_for(qt->fmt, qt->in_dim);
    if (!fast_ok(qt)) flags = XD_XT;
    ScratchPlan plan;
    plan.add(xdigits_bytes(seq, qt->in_dim, flags));
    std::vector<void *> ptrs;
    UT_TRY(scratch_acquire(ctx, plan, ptrs));
    ga.xd = xdigits_view(ptrs[0], seq, qt->in_dim, flags);
    UT_TRY(launch_digitize(ctx, x_dev, qt->in_dim, seq, qt->in_dim, nullptr, ga.xd, flags));
    return gemv(ctx, ga);
}

// QTensor::matvec_rows (qtensor.rs:548-586): the GEMV of one activation
// vector against the contiguous row block [row0, row0 + nrows), through a
// view of those rows (payload and scales offset, nothing copied).  For the
// integer formats each row's value is the one ut_qtensor_matmul gives for
// that row (exact integer sums); an f32 block may split K differently from
// the whole matrix, so its rows agree to rounding.
extern "C" int32_t ut_qtensor_matvec_rows(ut_ctx *ctx, const ut_qtensor *qt, int64_t row0,
                                          int64_t nrows, const float *x_dev, int64_t x_len,
                                          float *out_dev, int64_t out_len) {
    if (!ctx || !qt || !x_dev || (!out_dev && nrows > 0) || row0 < 0 || nrows < 0) {
        set_error(ctx, "ut_qtensor_matvec_rows: bad argument");
        return UT_ERR_ARG;
    }
    // the reference's assert!/assert_eq!s (qtensor.rs:549-552)
    if (row0 + nrows > qt->out_dim) {
        set_error(ctx, "rows [%lld, %lld) exceed out_dim %lld", (long long)row0,
                  (long long)(row0 + nrows), (long long)qt->out_dim);
        return UT_ERR_SHAPE;
    }
    if (x_len != qt->in_dim || out_len != nrows) {
        set_error(ctx, "matvec_rows shapes: x %lld (in %lld), out %lld (rows %lld)",
                  (long long)x_len, (long long)qt->in_dim, (long long)out_len, (long long)nrows);
        return UT_ERR_SHAPE;
    }
    if (nrows == 0) return UT_OK;
    ut_qtensor view = *qt;
    view.owns = false;
    view.out_dim = nrows;
    view.payload = (uint8_t *)qt->payload + row0 * qt->row_bytes;
    view.scales = qt->scales ? qt->scales + row0 : nullptr;
    return ut_qtensor_matmul(ctx, &view, out_dev, nrows, x_dev, qt->in_dim, 1);
}
