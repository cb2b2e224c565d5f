// ut_ops.hip -- embedding, rmsnorm, RoPE, residual adds and the MLA
// absorption products (adapters/undertow-deepseek-moe/src/{model,
// attention}.rs; undertow-quant/src/lib.rs).  Elementwise arithmetic keeps
// the reference's rounding: separate f32 multiplies and adds, no
// contraction, the reference's operation order.
#include "ut_ops.h"

namespace ut {


__global__ void k_embed(int32_t fmt, const uint8_t *__restrict__ payload,
                        const float *__restrict__ scales, int64_t row_bytes, int64_t H,
                        const int32_t *__restrict__ ids, float *__restrict__ out, int64_t ldo) {
    const int64_t s = blockIdx.y;
    const int64_t id = ids[s];
    const uint8_t *row = payload + id * row_bytes;
    // add_scaled_row(id, 1.0) into zeros: f = 1*scale; 0 + f*q
    const float f = fmt == UT_FMT_F32 ? 1.0f : __fmul_rn(1.0f, scales[id]);
#pragma unroll 8
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < H;
         i += (int64_t)gridDim.x * blockDim.x)
        out[s * ldo + i] = __fadd_rn(0.0f, __fmul_rn(f, code_at(fmt, row, i)));
}

int32_t launch_embed(ut_ctx *ctx, const ut_qtensor *emb, const int32_t *ids, int64_t rows,
                     float *out, int64_t ldo) {
    if (rows <= 0) return UT_OK;
    unsigned bx = (unsigned)((emb->in_dim + 255) / 256);
    if (bx > 64) bx = 64;
    int tok = timing_begin(ctx, "embed");
    hipLaunchKernelGGL(k_embed, dim3(bx, (unsigned)rows), dim3(256), 0, ctx->stream, emb->fmt,
                       (const uint8_t *)emb->payload, emb->scales, emb->row_bytes, emb->in_dim, ids,
                       out, ldo);
    timing_end(ctx, tok);
    return launch_check(ctx, "k_embed");
}

__global__ __launch_bounds__(256) void k_rmsnorm(const float *__restrict__ x, int64_t ldx,
                                                 const float *__restrict__ w, int64_t n, float eps,
                                                 float *__restrict__ out, int64_t ldo) {
    const int64_t s = blockIdx.x;
    const float *xr = x + s * ldx;
    __shared__ double red[4];
    double acc = 0.0;
#pragma unroll 8
    for (int64_t i = threadIdx.x; i < n; i += 256) {
        double v = (double)xr[i];
        acc += v * v;
    }
    for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    const double ms = ((red[0] + red[1]) + (red[2] + red[3])) / (double)n;
    const float r = 1.0f / sqrtf(__fadd_rn((float)ms, eps));
#pragma unroll 8
    for (int64_t i = threadIdx.x; i < n; i += 256)
        out[s * ldo + i] = __fmul_rn(__fmul_rn(xr[i], r), w[i]);
}

int32_t launch_rmsnorm(ut_ctx *ctx, const float *x, int64_t ldx, const float *w, int64_t n,
                       float eps, int64_t rows, float *out, int64_t ldo) {
    if (rows <= 0) return UT_OK;
    int tok = timing_begin(ctx, "rmsnorm");
    hipLaunchKernelGGL(k_rmsnorm, dim3((unsigned)rows), dim3(256), 0, ctx->stream, x, ldx, w, n,
                       eps, out, ldo);
    timing_end(ctx, tok);
    return launch_check(ctx, "k_rmsnorm");
}

__global__ void k_add(float *__restrict__ y, const float *__restrict__ x, int64_t n) {
#pragma unroll 8
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        y[i] = __fadd_rn(y[i], x[i]);
}

int32_t launch_add(ut_ctx *ctx, float *y, const float *x, int64_t n) {
    if (n <= 0) return UT_OK;
    unsigned blocks = (unsigned)((n + 255) / 256);
    if (blocks > 1024) blocks = 1024;
    int tok = timing_begin(ctx, "add");
    hipLaunchKernelGGL(k_add, dim3(blocks), dim3(256), 0, ctx->stream, y, x, n);
    timing_end(ctx, tok);
    return launch_check(ctx, "k_add");
}

__global__ void k_bf16_to_f32(const uint16_t *__restrict__ x, int64_t n, float *__restrict__ y) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        y[i] = __uint_as_float((uint32_t)x[i] << 16);
}

int32_t launch_bf16_to_f32(ut_ctx *ctx, const uint16_t *x, int64_t n, float *y) {
    if (n <= 0) return UT_OK;
    unsigned blocks = (unsigned)((n + 255) / 256);
    if (blocks > 1024) blocks = 1024;
    int tok = timing_begin(ctx, "bf16_to_f32");
    hipLaunchKernelGGL(k_bf16_to_f32, dim3(blocks), dim3(256), 0, ctx->stream, x, n, y);
    timing_end(ctx, tok);
    return launch_check(ctx, "k_bf16_to_f32");
}

// rows x H floats from src into dst rows pos.. (row stride ld): the
// pre-norm hidden states the MTP head reads later.
__global__ void k_copy_rows_at(float *__restrict__ dst, int64_t ld, PosRef pos,
                               const float *__restrict__ src, int64_t H) {
    float *d = dst + (pos.get() + blockIdx.y) * ld;
    const float *s = src + (int64_t)blockIdx.y * H;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < H;
         i += (int64_t)gridDim.x * blockDim.x)
        d[i] = s[i];
}

int32_t launch_copy_rows_at(ut_ctx *ctx, float *dst, int64_t ld, int64_t pos, const float *src,
                            int64_t rows, int64_t H) {
    if (rows <= 0) return UT_OK;
    unsigned bx = (unsigned)((H + 255) / 256);
    if (bx > 32) bx = 32;
    int tok = timing_begin(ctx, "copy_rows");
    hipLaunchKernelGGL(k_copy_rows_at, dim3(bx, (unsigned)rows), dim3(256), 0, ctx->stream, dst, ld,
                       pos_ref(ctx, pos), src, H);
    timing_end(ctx, tok);
    return launch_check(ctx, "k_copy_rows_at");
}

// Rows [pos, pos + rows) of src (row stride ld) into dst (rows x H): the
// MTP feed's hidden rows, read at a position the device word may hold.
__global__ void k_copy_rows_from(float *__restrict__ dst, const float *__restrict__ src, int64_t ld,
                                 PosRef pos, int64_t H) {
    const float *s = src + (pos.get() + blockIdx.y) * ld;
    float *d = dst + (int64_t)blockIdx.y * H;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < H;
         i += (int64_t)gridDim.x * blockDim.x)
        d[i] = s[i];
}

int32_t launch_copy_rows_from(ut_ctx *ctx, float *dst, const float *src, int64_t ld, int64_t pos,
                              int64_t rows, int64_t H) {
    if (rows <= 0) return UT_OK;
    unsigned bx = (unsigned)((H + 255) / 256);
    if (bx > 32) bx = 32;
    int tok = timing_begin(ctx, "copy_rows");
    hipLaunchKernelGGL(k_copy_rows_from, dim3(bx, (unsigned)rows), dim3(256), 0, ctx->stream, dst,
                       src, ld, pos_ref(ctx, pos), H);
    timing_end(ctx, tok);
    return launch_check(ctx, "k_copy_rows_from");
}

// The MTP feed's token ids after a verify of [next, d1..dk] that accepted
// `a` drafts (mtp.rs:84-121): the accepted drafts d1..da (vids[1..a]) and
// the verify's argmax row a (the next token), a + 1 ids into dst.
__global__ void k_feed_ids(int32_t *__restrict__ dst, const int32_t *__restrict__ vids,
                           const int32_t *__restrict__ am, int a) {
    const int i = threadIdx.x;
    if (i < a) dst[i] = vids[1 + i];
    else if (i == a) dst[i] = am[a];
}

int32_t launch_feed_ids(ut_ctx *ctx, int32_t *dst, const int32_t *vids, const int32_t *am, int a) {
    hipLaunchKernelGGL(k_feed_ids, dim3(1), dim3(64), 0, ctx->stream, dst, vids, am, a);
    return launch_check(ctx, "k_feed_ids");
}

// The device position word of a captured decode step: set before a replay
// when the host moved the position, advanced by the step itself.
__global__ void k_pos_set(int64_t *p, int64_t v) {
    if (threadIdx.x == 0) *p = v;
}
__global__ void k_pos_add(int64_t *p, int64_t n) {
    if (threadIdx.x == 0) *p += n;
}

int32_t launch_pos_set(ut_ctx *ctx, int64_t *p, int64_t v) {
    hipLaunchKernelGGL(k_pos_set, dim3(1), dim3(64), 0, ctx->stream, p, v);
    return launch_check(ctx, "k_pos_set");
}

int32_t launch_pos_add(ut_ctx *ctx, int64_t *p, int64_t n) {
    hipLaunchKernelGGL(k_pos_add, dim3(1), dim3(64), 0, ctx->stream, p, n);
    return launch_check(ctx, "k_pos_add");
}

// Cache append, one workgroup per row (kv_append_row).
__global__ __launch_bounds__(256) void k_kv_append(const float *__restrict__ comp, int64_t L,
                                                   int64_t P, const float *__restrict__ w,
                                                   float eps, float *__restrict__ latent,
                                                   float *__restrict__ krot, __bf16 *__restrict__ kc,
                                                   PosRef pos,
                                                   const float2 *__restrict__ table) {
    __shared__ double red[4];
    const int64_t s = blockIdx.x;
    kv_append_row(comp + s * (L + P), L, P, w, eps, latent, krot, kc, pos.get() + s, table, red);
}

int32_t launch_kv_append(ut_ctx *ctx, const float *comp, int64_t rows, int64_t L, int64_t P,
                         const float *w, float eps, float *latent, float *krot, __bf16 *kc,
                         int64_t pos_base, const float2 *table) {
    if (rows <= 0) return UT_OK;
    int tok = timing_begin(ctx, "kv_append");
    hipLaunchKernelGGL(k_kv_append, dim3((unsigned)rows), dim3(256), 0, ctx->stream, comp, L, P, w,
                       eps, latent, krot, kc, pos_ref(ctx, pos_base), table);
    timing_end(ctx, tok);
    return launch_check(ctx, "k_kv_append");
}

// Four consecutive codes of a row as floats (int4: 2 bytes, int8: 4 bytes,
// f32: 16 bytes).  col % 4 == 0.
template <int FMT>
__device__ __forceinline__ float4 codes4(const uint8_t *row, int64_t col) {
    if constexpr (FMT == UT_FMT_F32) {
        return *(const float4 *)(row + col * 4);
    } else if constexpr (FMT == UT_FMT_INT8) {
        const uint32_t w = *(const uint32_t *)(row + col);
        return make_float4((float)(int8_t)(w & 0xff), (float)(int8_t)((w >> 8) & 0xff),
                           (float)(int8_t)((w >> 16) & 0xff), (float)(int8_t)(w >> 24));
    } else {
        const uint32_t w = *(const uint16_t *)(row + col / 2);
        auto nib = [](uint32_t v) { return (float)((int)(v ^ 8) - 8); };
        return make_float4(nib(w & 0xf), nib((w >> 4) & 0xf), nib((w >> 8) & 0xf), nib((w >> 12) & 0xf));
    }
}

// qabs: one workgroup per (head, group of up to 4 query rows); thread t owns
// latent columns 4t..4t+3.  The head's nope rows are added in d order per
// column (add_scaled_row semantics), with the weight loads of 16 rows
// issued ahead of their use.
template <int FMT, int RB>
__global__ __launch_bounds__(128) void k_absorb_q(const uint8_t *__restrict__ w,
                                                  const float *__restrict__ scales,
                                                  int64_t row_bytes, int64_t L,
                                                  const float *__restrict__ q, int64_t rows,
                                                  int64_t heads, int64_t nope, int64_t rope,
                                                  int64_t kvh, float *__restrict__ qabs,
                                                  float *__restrict__ qrope, PosRef pos,
                                                  const float2 *__restrict__ table) {
    const int64_t pos_base = pos.get();
    const int64_t h = blockIdx.x, r0 = (int64_t)blockIdx.y * RB;
    const int64_t qh = nope + rope;
    const int64_t col = 512 * (int64_t)blockIdx.z + 4 * (int64_t)threadIdx.x;
    if (col < L) {
        float4 acc[RB];
#pragma unroll
        for (int r = 0; r < RB; r++) acc[r] = make_float4(0.f, 0.f, 0.f, 0.f);
        constexpr int U = 16;
        for (int64_t d0 = 0; d0 < nope; d0 += U) {
            float4 c[U];
#pragma unroll
            for (int u = 0; u < U; u++)
                if (d0 + u < nope) c[u] = codes4<FMT>(w + (h * kvh + d0 + u) * row_bytes, col);
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int64_t d = d0 + u;
                if (d >= nope) break;
                const float sc = FMT == UT_FMT_F32 ? 1.0f : scales[h * kvh + d];
#pragma unroll
                for (int r = 0; r < RB; r++) {
                    if (r0 + r >= rows) break;
                    const float qn = q[((r0 + r) * heads + h) * qh + d];
                    const float f = FMT == UT_FMT_F32 ? qn : __fmul_rn(qn, sc);
                    acc[r].x = __fadd_rn(acc[r].x, __fmul_rn(f, c[u].x));
                    acc[r].y = __fadd_rn(acc[r].y, __fmul_rn(f, c[u].y));
                    acc[r].z = __fadd_rn(acc[r].z, __fmul_rn(f, c[u].z));
                    acc[r].w = __fadd_rn(acc[r].w, __fmul_rn(f, c[u].w));
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RB; r++)
            if (r0 + r < rows) *(float4 *)(qabs + ((r0 + r) * heads + h) * L + col) = acc[r];
    }
    if (blockIdx.z == 0) {
        // q_rope = rope_interleave(q[nope:], pos_base + r) (attention.rs:106-118,156-166)
        const int64_t half = rope / 2;
        for (int64_t i = threadIdx.x; i < RB * rope; i += blockDim.x) {
            const int64_t r = r0 + i / rope, jj = i % rope;
            if (r >= rows) continue;
            const float *in = q + (r * heads + h) * qh + nope;
            const int64_t j = jj < half ? jj : jj - half;
            const float a = in[2 * j], b = in[2 * j + 1];
            const float2 cs = table[(pos_base + r) * half + j];
            qrope[(r * heads + h) * rope + jj] =
                jj < half ? __fsub_rn(__fmul_rn(a, cs.x), __fmul_rn(b, cs.y))
                          : __fadd_rn(__fmul_rn(b, cs.x), __fmul_rn(a, cs.y));
        }
    }
}

// The same product with the head's nope rows staged in LDS first: a
// workgroup takes one head, one block of CB latent columns and up to 4
// query rows.  All of the block's weight bytes are requested at once
// (16-byte loads, a few per thread), then thread t adds the nope rows of
// column t in d order from LDS.  f[r][d] = q*scale is formed once in LDS.
template <int FMT, int RB, int CB>
__global__ __launch_bounds__(CB) void k_absorb_q_lds(const uint8_t *__restrict__ w,
                                                     const float *__restrict__ scales,
                                                     int64_t row_bytes, int64_t L,
                                                     const float *__restrict__ q, int64_t rows,
                                                     int64_t heads, int nope, int64_t rope,
                                                     int64_t kvh, float *__restrict__ qabs,
                                                     float *__restrict__ qrope, PosRef pos,
                                                     const float2 *__restrict__ table) {
    const int64_t pos_base = pos.get();
    constexpr int BPC2 = FMT == UT_FMT_INT4 ? 1 : FMT == UT_FMT_INT8 ? 2 : 8;  // 2*bytes/col
    constexpr int ROWB = CB * BPC2 / 2;  // staged bytes per nope row
    constexpr int PIECES = ROWB / 16;
    extern __shared__ __attribute__((aligned(16))) uint8_t sm_abs[];
    uint8_t *codes = sm_abs;                                   // [nope][ROWB]
    float *f = (float *)(sm_abs + (size_t)nope * ROWB);       // [RB][nope]
    const int64_t h = blockIdx.x, r0 = (int64_t)blockIdx.z * RB;
    const int64_t qh = nope + rope;
    const int tid = threadIdx.x;
    const int64_t cb0 = (int64_t)blockIdx.y * CB;
    const uint8_t *wh = w + (h * kvh) * row_bytes + cb0 * BPC2 / 2;
    for (int i = tid; i < nope * PIECES; i += CB) {
        const int d = i / PIECES, pc = i - d * PIECES;
        *(uint4 *)(codes + d * ROWB + 16 * pc) = *(const uint4 *)(wh + d * row_bytes + 16 * pc);
    }
    for (int i = tid; i < RB * nope; i += CB) {
        const int r = i / nope, d = i - r * nope;
        const int64_t rr = r0 + r < rows ? r0 + r : rows - 1;
        const float qn = q[(rr * heads + h) * qh + d];
        f[i] = FMT == UT_FMT_F32 ? qn : __fmul_rn(qn, scales[h * kvh + d]);
    }
    __syncthreads();
    float acc[RB];
#pragma unroll
    for (int r = 0; r < RB; r++) acc[r] = 0.0f;
#pragma unroll 8
    for (int d = 0; d < nope; d++) {
        float c;
        if constexpr (FMT == UT_FMT_F32) {
            c = *(const float *)(codes + d * ROWB + 4 * tid);
        } else if constexpr (FMT == UT_FMT_INT8) {
            c = (float)(int8_t)codes[d * ROWB + tid];
        } else {
            const uint32_t b = codes[d * ROWB + (tid >> 1)];
            c = (float)((int)(((b >> (4 * (tid & 1))) & 0xf) ^ 8) - 8);
        }
#pragma unroll
        for (int r = 0; r < RB; r++) acc[r] = __fadd_rn(acc[r], __fmul_rn(f[r * nope + d], c));
    }
#pragma unroll
    for (int r = 0; r < RB; r++)
        if (r0 + r < rows) qabs[((r0 + r) * heads + h) * L + cb0 + tid] = acc[r];
    if (blockIdx.y == 0) {
        // q_rope = rope_interleave(q[nope:], pos_base + r) (attention.rs:106-118,156-166)
        const int64_t half = rope / 2;
        for (int64_t i = tid; i < RB * rope; i += CB) {
            const int64_t r = r0 + i / rope, jj = i % rope;
            if (r >= rows) continue;
            const float *in = q + (r * heads + h) * qh + nope;
            const int64_t j = jj < half ? jj : jj - half;
            const float a = in[2 * j], b = in[2 * j + 1];
            const float2 cs = table[(pos_base + r) * half + j];
            qrope[(r * heads + h) * rope + jj] =
                jj < half ? __fsub_rn(__fmul_rn(a, cs.x), __fmul_rn(b, cs.y))
                          : __fadd_rn(__fmul_rn(b, cs.x), __fmul_rn(a, cs.y));
        }
    }
}

template <int FMT, int RB, int CB>
static void absorb_q_lds_launch(ut_ctx *ctx, const ut_qtensor *kv_b, const float *q, int64_t rows,
                                int64_t heads, int64_t nope, int64_t rope, int64_t kvh,
                                float *qabs, float *qrope, int64_t pos_base,
                                const float2 *table) {
    const int64_t L = kv_b->in_dim;
    constexpr int BPC2 = FMT == UT_FMT_INT4 ? 1 : FMT == UT_FMT_INT8 ? 2 : 8;
    const size_t shmem = (size_t)nope * (CB * BPC2 / 2) + (size_t)RB * nope * 4;
    dim3 grid((unsigned)heads, (unsigned)(L / CB), (unsigned)((rows + RB - 1) / RB));
    hipLaunchKernelGGL((k_absorb_q_lds<FMT, RB, CB>), grid, dim3(CB), shmem, ctx->stream,
                       (const uint8_t *)kv_b->payload, kv_b->scales, kv_b->row_bytes, L, q, rows,
                       heads, (int)nope, rope, kvh, qabs, qrope, pos_ref(ctx, pos_base), table);
}

int32_t launch_absorb_q(ut_ctx *ctx, const ut_qtensor *kv_b, const float *q, int64_t rows,
                        int64_t heads, int64_t nope, int64_t rope, int64_t vh, float *qabs,
                        float *qrope, int64_t pos_base, const float2 *table) {
    if (rows <= 0) return UT_OK;
    const int64_t L = kv_b->in_dim;
    if (L % 4 != 0) {
        set_error(ctx, "absorb: kv_lora_rank %lld must be a multiple of 4", (long long)L);
        return UT_ERR_SHAPE;
    }
    constexpr int RB = 4;
    const int64_t kvh = nope + vh;
    // LDS-staged kernel: 128- (or 64-) column blocks, 16-byte aligned rows,
    // the block's nope rows within 64 KiB of LDS
    const int bpc2 = kv_b->fmt == UT_FMT_INT4 ? 1 : kv_b->fmt == UT_FMT_INT8 ? 2 : 8;
    const int cb = L % 128 == 0 ? 128 : L % 64 == 0 ? 64 : 0;
    if (cb && (cb * bpc2 / 2) % 16 == 0 && kv_b->row_bytes % 16 == 0 &&
        ((uintptr_t)kv_b->payload & 15) == 0 &&
        (size_t)nope * (cb * bpc2 / 2) + RB * nope * 4 <= 64 * 1024) {
        int tok = timing_begin(ctx, "absorb_q");
        // query rows per pass: as many as are there, up to RB (the rows ride
        // along in the same loop; a single decode row does a quarter of the work)
#define UT_ABSQ(F, C)                                                                                   \
    do {                                                                                                \
        if (rows == 1) absorb_q_lds_launch<F, 1, C>(ctx, kv_b, q, rows, heads, nope, rope, kvh, qabs, qrope, pos_base, table); \
        else if (rows == 2) absorb_q_lds_launch<F, 2, C>(ctx, kv_b, q, rows, heads, nope, rope, kvh, qabs, qrope, pos_base, table); \
        else absorb_q_lds_launch<F, RB, C>(ctx, kv_b, q, rows, heads, nope, rope, kvh, qabs, qrope, pos_base, table); \
    } while (0)
        if (cb == 128) {
            if (kv_b->fmt == UT_FMT_INT8) UT_ABSQ(UT_FMT_INT8, 128);
            else if (kv_b->fmt == UT_FMT_INT4) UT_ABSQ(UT_FMT_INT4, 128);
            else UT_ABSQ(UT_FMT_F32, 128);
        } else {
            if (kv_b->fmt == UT_FMT_INT8) UT_ABSQ(UT_FMT_INT8, 64);
            else if (kv_b->fmt == UT_FMT_INT4) UT_ABSQ(UT_FMT_INT4, 64);
            else UT_ABSQ(UT_FMT_F32, 64);
        }
#undef UT_ABSQ
        timing_end(ctx, tok);
        return launch_check(ctx, "k_absorb_q_lds");
    }
    // 128 threads x 4 columns per workgroup column block
    const unsigned threads = (unsigned)(L >= 512 ? 128 : ((L / 4) + 63) / 64 * 64);
    dim3 grid((unsigned)heads, (unsigned)((rows + RB - 1) / RB), (unsigned)((L + 511) / 512));
    const uint8_t *w = (const uint8_t *)kv_b->payload;
    int tok = timing_begin(ctx, "absorb_q");
    switch (kv_b->fmt) {
    case UT_FMT_INT8: hipLaunchKernelGGL((k_absorb_q<UT_FMT_INT8, RB>), grid, dim3(threads), 0, ctx->stream, w, kv_b->scales, kv_b->row_bytes, L, q, rows, heads, nope, rope, kvh, qabs, qrope, pos_ref(ctx, pos_base), table); break;
    case UT_FMT_INT4: hipLaunchKernelGGL((k_absorb_q<UT_FMT_INT4, RB>), grid, dim3(threads), 0, ctx->stream, w, kv_b->scales, kv_b->row_bytes, L, q, rows, heads, nope, rope, kvh, qabs, qrope, pos_ref(ctx, pos_base), table); break;
    default: hipLaunchKernelGGL((k_absorb_q<UT_FMT_F32, RB>), grid, dim3(threads), 0, ctx->stream, w, kv_b->scales, kv_b->row_bytes, L, q, rows, heads, nope, rope, kvh, qabs, qrope, pos_ref(ctx, pos_base), table); break;
    }
    timing_end(ctx, tok);
    return launch_check(ctx, "k_absorb_q");
}

// ctx values: one workgroup per (head, 16 output rows j, group of up to 4
// query rows); 16 sub-lanes per row each take L/16 columns in 4-column
// pieces, then a fixed butterfly.  The value of (row r, output j) is read
// from sub-lane r, whatever the number of query rows.
template <int FMT, int RB>
__global__ __launch_bounds__(256) void k_absorb_v(const uint8_t *__restrict__ w,
                                                  const float *__restrict__ scales,
                                                  int64_t row_bytes, int64_t L,
                                                  const float *__restrict__ clat, int64_t rows,
                                                  int64_t heads, int64_t nope, int64_t vh,
                                                  float *__restrict__ out) {
    const int64_t h = blockIdx.x, r0 = (int64_t)blockIdx.z * RB;
    const int jl = threadIdx.x >> 4, s = threadIdx.x & 15;
    const int64_t j = (int64_t)blockIdx.y * 16 + jl;
    const int64_t jc = j < vh ? j : vh - 1;
    const int64_t row = h * (nope + vh) + nope + jc;
    const uint8_t *wr = w + row * row_bytes;
    float acc[RB];
#pragma unroll
    for (int r = 0; r < RB; r++) acc[r] = 0.0f;
#pragma unroll 8
    for (int64_t c = 4 * s; c < L; c += 64) {
        const float4 cw = codes4<FMT>(wr, c);
#pragma unroll
        for (int r = 0; r < RB; r++) {
            const int64_t rr = r0 + r < rows ? r0 + r : rows - 1;
            const float4 xv = *(const float4 *)(clat + (rr * heads + h) * L + c);
            float a = acc[r];
            a = __builtin_fmaf(xv.x, cw.x, a);
            a = __builtin_fmaf(xv.y, cw.y, a);
            a = __builtin_fmaf(xv.z, cw.z, a);
            a = __builtin_fmaf(xv.w, cw.w, a);
            acc[r] = a;
        }
    }
#pragma unroll
    for (int r = 0; r < RB; r++) {
        float v = acc[r];
#pragma unroll
        for (int off = 8; off >= 1; off >>= 1) v += __shfl_xor(v, off, 16);
        if (s == r && j < vh && r0 + r < rows)
            out[(r0 + r) * heads * vh + h * vh + j] = FMT == UT_FMT_F32 ? v : __fmul_rn(v, scales[row]);
    }
}

// int8 weights, latent width 512: 32 lanes per output row, lane k takes
// columns 16k..16k+15 with one 16-byte code load, then a butterfly over the
// 32 lanes; a workgroup covers NP passes of 8 output rows of one head, with
// the head's RB context rows staged in LDS once (every output row reads
// them).
// vmax (optional): per row, this workgroup's max |out| (float bits) at
// [row][h * gridDim.y + blockIdx.y], for a consumer that digitises the row
// (absorb_v_parts per row).  Two passes per workgroup (config-4 verify of
// four rows: 10.9 -> 8.4 us; o_proj, which reduces the maxima while it
// stages, 32.6 -> 30.8 us); one pass and four measured slower.
constexpr int kAbsorbVPasses = 2;
template <int RB, int NP>
__global__ __launch_bounds__(256) void k_absorb_v_i8(const uint8_t *__restrict__ w,
                                                         const float *__restrict__ scales,
                                                         int64_t row_bytes,
                                                         const float *__restrict__ clat,
                                                         int64_t rows, int64_t heads, int64_t nope,
                                                         int64_t vh, float *__restrict__ out,
                                                         uint32_t *__restrict__ vmax) {
    constexpr int L = 512;
    __shared__ __attribute__((aligned(16))) float sx[RB][L];
    __shared__ uint32_t smax[RB][8 * NP];
    const int64_t h = blockIdx.x, r0 = (int64_t)blockIdx.z * RB;
    const int tid = threadIdx.x, jl = tid >> 5, k = tid & 31;
    uint4 cw[NP];
    int64_t wrow[NP];
#pragma unroll
    for (int p = 0; p < NP; p++) {
        const int64_t j = ((int64_t)blockIdx.y * NP + p) * 8 + jl;
        const int64_t jc = j < vh ? j : vh - 1;
        wrow[p] = h * (nope + vh) + nope + jc;
        cw[p] = *(const uint4 *)(w + wrow[p] * row_bytes + 16 * k);
    }
    for (int i = tid; i < RB * (L / 4); i += 256) {
        const int r = i / (L / 4), q = i - r * (L / 4);
        const int64_t rr = r0 + r < rows ? r0 + r : rows - 1;
        *(float4 *)&sx[r][4 * q] = *(const float4 *)(clat + (rr * heads + h) * L + 4 * q);
    }
    __syncthreads();
#pragma unroll
    for (int p = 0; p < NP; p++) {
        const int64_t j = ((int64_t)blockIdx.y * NP + p) * 8 + jl;
        float acc[RB];
#pragma unroll
        for (int r = 0; r < RB; r++) {
            const float *xr = &sx[r][16 * k];
            float a = 0.0f;
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++) {
                const float4 xv = *(const float4 *)(xr + 4 * q4);
                const uint32_t word = q4 == 0 ? cw[p].x : q4 == 1 ? cw[p].y : q4 == 2 ? cw[p].z : cw[p].w;
                a = __builtin_fmaf(xv.x, (float)(int8_t)(word), a);
                a = __builtin_fmaf(xv.y, (float)(int8_t)(word >> 8), a);
                a = __builtin_fmaf(xv.z, (float)(int8_t)(word >> 16), a);
                a = __builtin_fmaf(xv.w, (float)(int8_t)(word >> 24), a);
            }
#pragma unroll
            for (int off = 16; off >= 1; off >>= 1) a += __shfl_xor(a, off, 32);
            acc[r] = a;
        }
#pragma unroll
        for (int r = 0; r < RB; r++) {
            const float v = __fmul_rn(acc[r], scales[wrow[p]]);
            if (k == r) smax[r][p * 8 + jl] = j < vh ? __float_as_uint(fabsf(v)) : 0u;
            if (k == r && j < vh && r0 + r < rows) out[(r0 + r) * heads * vh + h * vh + j] = v;
        }
    }
    if (vmax) {
        __syncthreads();
        if (tid < RB && r0 + tid < rows) {
            uint32_t mx = smax[tid][0];
#pragma unroll
            for (int q = 1; q < 8 * NP; q++) mx = max(mx, smax[tid][q]);
            const int64_t nparts = heads * (int64_t)gridDim.y;
            vmax[(r0 + tid) * nparts + h * gridDim.y + blockIdx.y] = mx;
        }
    }
}

int64_t absorb_v_parts(int64_t heads, int64_t vh) {
    constexpr int64_t rows_per_wg = 8 * kAbsorbVPasses;
    return heads * ((vh + rows_per_wg - 1) / rows_per_wg);
}

bool absorb_v_max_ok(const ut_qtensor *kv_b) {
    return kv_b->fmt == UT_FMT_INT8 && kv_b->in_dim == 512 && kv_b->row_bytes % 16 == 0 &&
           ((uintptr_t)kv_b->payload & 15) == 0;
}

int32_t launch_absorb_v(ut_ctx *ctx, const ut_qtensor *kv_b, const float *clat, int64_t rows,
                        int64_t heads, int64_t nope, int64_t vh, float *out, uint32_t *vmax) {
    if (vmax && !absorb_v_max_ok(kv_b)) {
        set_error(ctx, "absorb_v: row maxima need the int8 512-wide kernel");
        return UT_ERR_ARG;
    }
    if (rows <= 0) return UT_OK;
    const int64_t L = kv_b->in_dim;
    if (L % 4 != 0) {
        set_error(ctx, "absorb: kv_lora_rank %lld must be a multiple of 4", (long long)L);
        return UT_ERR_SHAPE;
    }
    constexpr int RB = 4;
    const uint8_t *w = (const uint8_t *)kv_b->payload;
    if (kv_b->fmt == UT_FMT_INT8 && L == 512 && kv_b->row_bytes % 16 == 0 &&
        ((uintptr_t)w & 15) == 0) {
        int tok = timing_begin(ctx, "absorb_v");
        constexpr int NP = kAbsorbVPasses;
        const dim3 g((unsigned)heads, (unsigned)((vh + 8 * NP - 1) / (8 * NP)),
                     (unsigned)((rows + RB - 1) / RB));
        if (rows == 1)
            hipLaunchKernelGGL((k_absorb_v_i8<1, NP>), g, dim3(256), 0, ctx->stream, w,
                               kv_b->scales, kv_b->row_bytes, clat, rows, heads, nope, vh, out, vmax);
        else if (rows == 2)
            hipLaunchKernelGGL((k_absorb_v_i8<2, NP>), g, dim3(256), 0, ctx->stream, w,
                               kv_b->scales, kv_b->row_bytes, clat, rows, heads, nope, vh, out, vmax);
        else
            hipLaunchKernelGGL((k_absorb_v_i8<RB, NP>), g, dim3(256), 0, ctx->stream, w,
                               kv_b->scales, kv_b->row_bytes, clat, rows, heads, nope, vh, out, vmax);
        timing_end(ctx, tok);
        return launch_check(ctx, "k_absorb_v_i8");
    }
    dim3 grid((unsigned)heads, (unsigned)((vh + 15) / 16), (unsigned)((rows + RB - 1) / RB));
    int tok = timing_begin(ctx, "absorb_v");
    switch (kv_b->fmt) {
    case UT_FMT_INT8: hipLaunchKernelGGL((k_absorb_v<UT_FMT_INT8, RB>), grid, dim3(256), 0, ctx->stream, w, kv_b->scales, kv_b->row_bytes, L, clat, rows, heads, nope, vh, out); break;
    case UT_FMT_INT4: hipLaunchKernelGGL((k_absorb_v<UT_FMT_INT4, RB>), grid, dim3(256), 0, ctx->stream, w, kv_b->scales, kv_b->row_bytes, L, clat, rows, heads, nope, vh, out); break;
    default: hipLaunchKernelGGL((k_absorb_v<UT_FMT_F32, RB>), grid, dim3(256), 0, ctx->stream, w, kv_b->scales, kv_b->row_bytes, L, clat, rows, heads, nope, vh, out); break;
    }
    timing_end(ctx, tok);
    return launch_check(ctx, "k_absorb_v");
}

}  // namespace ut
