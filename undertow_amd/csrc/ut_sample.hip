// ut_sample.hip -- greedy argmax over logits rows (undertow-core/src/
// sample.rs:353-361): the first index of the maximum, NaN never selected,
// and 0 when row[0] is NaN (no `x > NaN` compare succeeds).
//
// Two launches: k_argmax_partial splits each row over many workgroups
// (vocab 129280 rows are read at full bandwidth), k_argmax_final reduces
// the partials.  Ties keep the lowest index; the result does not depend
// on the split.
#include "ut_argmax.h"
#include "ut_internal.h"
#include "ut_sample.h"

namespace ut {

__global__ __launch_bounds__(256) void k_argmax_partial(const float *__restrict__ x, int64_t V,
                                                        int64_t ldx, int64_t chunk,
                                                        float *__restrict__ pv,
                                                        int32_t *__restrict__ pi) {
    const int64_t row = blockIdx.y;
    const float *xr = x + row * ldx;
    const int64_t lo = (int64_t)blockIdx.x * chunk, hi = lo + chunk < V ? lo + chunk : V;
    Best b{0.0f, -1};
#pragma unroll 8
    for (int64_t i = lo + threadIdx.x; i < hi; i += blockDim.x) {
        float v = xr[i];
        if (v == v && (b.i < 0 || v > b.v)) { b.v = v; b.i = (int32_t)i; }
    }
    b = block_best(b);
    if (threadIdx.x == 0) {
        pv[row * gridDim.x + blockIdx.x] = b.v;
        pi[row * gridDim.x + blockIdx.x] = b.i;
    }
}

// One workgroup per row: the best of the row's nparts partials, then the
// row rule (index 0 when x[row][0] is NaN or nothing was a candidate).
// err: also copies the sticky error word to idx[rows] (one readback for both).
__global__ __launch_bounds__(256) void k_argmax_final(const float *__restrict__ x, int64_t ldx,
                                                      int64_t nparts, const float *__restrict__ pv,
                                                      const int32_t *__restrict__ pi,
                                                      int32_t *__restrict__ idx,
                                                      const int32_t *__restrict__ err,
                                                      const int32_t *__restrict__ tail, int ntail) {
    const int64_t row = blockIdx.x;
    Best b{0.0f, -1};
    // 16 partials per thread per round, every load of a round issued first
    constexpr int U = 16;
    for (int64_t j0 = 0; j0 < nparts; j0 += U * (int64_t)blockDim.x) {
        Best c[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int64_t j = j0 + threadIdx.x + (int64_t)u * blockDim.x;
            c[u] = j < nparts ? Best{pv[row * nparts + j], pi[row * nparts + j]} : Best{0.0f, -1};
        }
#pragma unroll
        for (int u = 0; u < U; u++) b = better(b, c[u]);
    }
    b = block_best(b);
    if (threadIdx.x == 0) {
        const float x0 = x[row * ldx];
        idx[row] = (x0 != x0 || b.i < 0) ? 0 : b.i;
        if (err && row == (int64_t)gridDim.x - 1) idx[gridDim.x] = *err;
    }
    // after the error word, ntail ints of tail (a verify step's draft ids),
    // so that one readback carries all three
    if (err && tail && row == (int64_t)gridDim.x - 1 && (int)threadIdx.x < ntail)
        idx[gridDim.x + 1 + threadIdx.x] = tail[threadIdx.x];
}

size_t argmax_scratch_bytes(int64_t rows, int64_t V) {
    // the widest partial set: a GEMV epilogue's, one per 16 output rows
    int64_t parts = argmax_parts(V);
    const int64_t gemv_parts = argmax_gemv_parts_max(V);
    if (gemv_parts > parts) parts = gemv_parts;
    return (size_t)rows * parts * 8 + 512;
}

int64_t argmax_gemv_parts_max(int64_t V) { return (V + 15) / 16; }

ArgmaxParts argmax_parts_view(void *scratch, int64_t rows, int64_t stride) {
    ArgmaxParts p;
    p.v = (float *)scratch;
    p.i = (int32_t *)((char *)scratch + ((rows * stride * 4 + 255) & ~int64_t(255)));
    p.stride = stride;
    return p;
}

int32_t launch_argmax_final(ut_ctx *ctx, const float *x, int64_t rows, int64_t ldx,
                            const ArgmaxParts &p, int32_t *idx, const int32_t *err,
                            const int32_t *tail, int ntail) {
    if (rows <= 0) return UT_OK;
    if (ntail < 0 || ntail > 256) {
        set_error(ctx, "argmax: %d tail ints (at most 256)", ntail);
        return UT_ERR_ARG;
    }
    int tok = timing_begin(ctx, "argmax_final");
    hipLaunchKernelGGL(k_argmax_final, dim3((unsigned)rows), dim3(256), 0, ctx->stream, x, ldx,
                       p.stride, p.v, p.i, idx, err, tail, ntail);
    timing_end(ctx, tok);
    return launch_check(ctx, "k_argmax_final");
}

int64_t argmax_parts(int64_t V) {
    int64_t p = (V + 4095) / 4096;
    if (p < 1) p = 1;
    if (p > 64) p = 64;
    return p;
}

int32_t launch_argmax(ut_ctx *ctx, const float *x, int64_t rows, int64_t V, int64_t ldx,
                      int32_t *idx, void *scratch, const int32_t *err, const int32_t *tail,
                      int ntail) {
    if (rows <= 0) return UT_OK;
    const int64_t parts = argmax_parts(V);
    const int64_t chunk = (V + parts - 1) / parts;
    const ArgmaxParts p = argmax_parts_view(scratch, rows, parts);
    int tok = timing_begin(ctx, "argmax");
    hipLaunchKernelGGL(k_argmax_partial, dim3((unsigned)parts, (unsigned)rows), dim3(256), 0,
                       ctx->stream, x, V, ldx, chunk, p.v, p.i);
    UT_TRY(launch_check(ctx, "k_argmax_partial"));
    timing_end(ctx, tok);
    return launch_argmax_final(ctx, x, rows, ldx, p, idx, err, tail, ntail);
}

}  // namespace ut

using namespace ut;

extern "C" int32_t ut_argmax_rows(ut_ctx *ctx, const float *logits_dev, int64_t rows,
                                  int64_t vocab, int32_t *idx_dev) {
    if (!ctx || !logits_dev || !idx_dev || rows < 0 || vocab <= 0 || vocab > INT32_MAX) {
        set_error(ctx, "ut_argmax_rows: bad argument");
        return UT_ERR_ARG;
    }
    if (rows == 0) return UT_OK;
    ScratchPlan plan;
    plan.add(argmax_scratch_bytes(rows, vocab) + 256);
    std::vector<void *> ptrs;
    UT_TRY(scratch_acquire(ctx, plan, ptrs));
    return launch_argmax(ctx, logits_dev, rows, vocab, vocab, idx_dev, ptrs[0]);
}
