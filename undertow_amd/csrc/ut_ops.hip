// ut_ops.hip -- embedding, rmsnorm, RoPE, residual adds and the MLA
// absorption products (adapters/undertow-deepseek-moe/src/{model,
// attention}.rs; undertow-quant/src/lib.rs).  Elementwise arithmetic keeps
// the reference's rounding: separate f32 multiplies and adds, no
// contraction, the reference's operation order.
#include "ut_ops.h"

namespace ut {

__device__ __forceinline__ float code_at(int32_t fmt, const uint8_t *row, int64_t i) {
    if (fmt == UT_FMT_F32) return ((const float *)row)[i];
    if (fmt == UT_FMT_INT8) return (float)(int8_t)row[i];
    uint8_t b = row[i >> 1];
    int nib = (i & 1) ? (b >> 4) : (b & 0xF);
    return (float)((nib ^ 8) - 8);
}

__global__ void k_embed(int32_t fmt, const uint8_t *__restrict__ payload,
                        const float *__restrict__ scales, int64_t row_bytes, int64_t H,
                        const int32_t *__restrict__ ids, float *__restrict__ out, int64_t ldo) {
    const int64_t s = blockIdx.y;
    const int64_t id = ids[s];
    const uint8_t *row = payload + id * row_bytes;
    // add_scaled_row(id, 1.0) into zeros: f = 1*scale; 0 + f*q
    const float f = fmt == UT_FMT_F32 ? 1.0f : __fmul_rn(1.0f, scales[id]);
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
    for (int64_t i = threadIdx.x; i < n; i += 256) {
        double v = (double)xr[i];
        acc += v * v;
    }
    for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    const double ms = ((red[0] + red[1]) + (red[2] + red[3])) / (double)n;
    const float r = 1.0f / sqrtf(__fadd_rn((float)ms, eps));
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

// One workgroup per (row, head) slice; the slice is read completely before
// any element is written (the permutation moves pairs to split halves).
__global__ void k_rope(float *__restrict__ v, int64_t heads, int64_t ld_row, int64_t ld_head,
                       int64_t dim, int64_t pos_base, const float2 *__restrict__ table,
                       int64_t table_stride) {
    const int64_t s = blockIdx.x / heads, h = blockIdx.x % heads;
    float *p = v + s * ld_row + h * ld_head;
    const int64_t half = dim / 2;
    const float2 *cs = table + (pos_base + s) * table_stride;
    const int j = threadIdx.x;
    float a = 0.0f, b = 0.0f;
    if (j < half) { a = p[2 * j]; b = p[2 * j + 1]; }
    __syncthreads();
    if (j < half) {
        const float c = cs[j].x, sn = cs[j].y;
        p[j] = __fsub_rn(__fmul_rn(a, c), __fmul_rn(b, sn));
        p[half + j] = __fadd_rn(__fmul_rn(b, c), __fmul_rn(a, sn));
    }
}

int32_t launch_rope(ut_ctx *ctx, float *v, int64_t rows, int64_t heads, int64_t ld_row,
                    int64_t ld_head, int64_t dim, int64_t pos_base, const float2 *table,
                    int64_t table_stride) {
    if (rows <= 0 || dim <= 0) return UT_OK;
    if (dim / 2 > 1024) {
        set_error(ctx, "rope dim %lld too large", (long long)dim);
        return UT_ERR_SHAPE;
    }
    unsigned threads = (unsigned)(((dim / 2) + 63) / 64 * 64);
    int tok = timing_begin(ctx, "rope");
    hipLaunchKernelGGL(k_rope, dim3((unsigned)(rows * heads)), dim3(threads), 0, ctx->stream, v,
                       heads, ld_row, ld_head, dim, pos_base, table, table_stride);
    timing_end(ctx, tok);
    return launch_check(ctx, "k_rope");
}

__global__ void k_add(float *__restrict__ y, const float *__restrict__ x, int64_t n) {
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

// qabs: one workgroup per (row, head), threads over the latent columns;
// the nope rows of the head are added in order (add_scaled_row semantics).
__global__ __launch_bounds__(256) void k_absorb_q(int32_t fmt, const uint8_t *__restrict__ w,
                                                  const float *__restrict__ scales,
                                                  int64_t row_bytes, int64_t L,
                                                  const float *__restrict__ q, int64_t heads,
                                                  int64_t nope, int64_t rope, int64_t kvh,
                                                  float *__restrict__ qabs,
                                                  float *__restrict__ qrope) {
    const int64_t sh = blockIdx.x;  // s*heads + h
    const int64_t h = sh % heads;
    const float *qn = q + sh * (nope + rope);
    for (int64_t i = threadIdx.x; i < L; i += 256) {
        float acc = 0.0f;
        for (int64_t d = 0; d < nope; d++) {
            const int64_t row = h * kvh + d;
            const float f = fmt == UT_FMT_F32 ? qn[d] : __fmul_rn(qn[d], scales[row]);
            acc = __fadd_rn(acc, __fmul_rn(f, code_at(fmt, w + row * row_bytes, i)));
        }
        qabs[sh * L + i] = acc;
    }
    for (int64_t i = threadIdx.x; i < rope; i += 256) qrope[sh * rope + i] = qn[nope + i];
}

int32_t launch_absorb_q(ut_ctx *ctx, const ut_qtensor *kv_b, const float *q, int64_t rows,
                        int64_t heads, int64_t nope, int64_t rope, int64_t vh, float *qabs,
                        float *qrope) {
    if (rows <= 0) return UT_OK;
    int tok = timing_begin(ctx, "absorb_q");
    hipLaunchKernelGGL(k_absorb_q, dim3((unsigned)(rows * heads)), dim3(256), 0, ctx->stream,
                       kv_b->fmt, (const uint8_t *)kv_b->payload, kv_b->scales, kv_b->row_bytes,
                       kv_b->in_dim, q, heads, nope, rope, nope + vh, qabs, qrope);
    timing_end(ctx, tok);
    return launch_check(ctx, "k_absorb_q");
}

// ctx values: one wave per (row, head, output j); lanes split the latent
// columns, then a fixed butterfly.
__global__ __launch_bounds__(256) void k_absorb_v(int32_t fmt, const uint8_t *__restrict__ w,
                                                  const float *__restrict__ scales,
                                                  int64_t row_bytes, int64_t L,
                                                  const float *__restrict__ clat, int64_t heads,
                                                  int64_t nope, int64_t vh,
                                                  float *__restrict__ out) {
    const int64_t sh = blockIdx.x;
    const int64_t h = sh % heads, s = sh / heads;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const float *x = clat + sh * L;
    for (int64_t j = wave; j < vh; j += 4) {
        const int64_t row = h * (nope + vh) + nope + j;
        const uint8_t *wr = w + row * row_bytes;
        float acc = 0.0f;
        for (int64_t i = lane; i < L; i += 64) acc = __builtin_fmaf(x[i], code_at(fmt, wr, i), acc);
        for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
        acc = __shfl(acc, 0, 64);
        if (lane == 0) out[s * heads * vh + h * vh + j] = fmt == UT_FMT_F32 ? acc : __fmul_rn(acc, scales[row]);
    }
}

int32_t launch_absorb_v(ut_ctx *ctx, const ut_qtensor *kv_b, const float *clat, int64_t rows,
                        int64_t heads, int64_t nope, int64_t vh, float *out) {
    if (rows <= 0) return UT_OK;
    int tok = timing_begin(ctx, "absorb_v");
    hipLaunchKernelGGL(k_absorb_v, dim3((unsigned)(rows * heads)), dim3(256), 0, ctx->stream,
                       kv_b->fmt, (const uint8_t *)kv_b->payload, kv_b->scales, kv_b->row_bytes,
                       kv_b->in_dim, clat, heads, nope, vh, out);
    timing_end(ctx, tok);
    return launch_check(ctx, "k_absorb_v");
}

}  // namespace ut
