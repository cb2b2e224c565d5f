// ut_sample.hip -- greedy argmax over logits rows (undertow-core/src/
// sample.rs:353-361): the first index of the maximum, NaN never selected,
// and 0 when row[0] is NaN (no `x > NaN` compare succeeds).
//
// Two launches: k_argmax_partial splits each row over many workgroups
// (vocab 129280 rows are read at full bandwidth), k_argmax_final reduces
// the partials.  Ties keep the lowest index; the result does not depend
// on the split.
#include "ut_internal.h"
#include "ut_sample.h"

namespace ut {

struct Best {
    float v;
    int32_t i;  // -1: no candidate
};

__device__ __forceinline__ Best better(Best a, Best b) {
    if (a.i < 0) return b;
    if (b.i < 0) return a;
    if (b.v > a.v || (b.v == a.v && b.i < a.i)) return b;
    return a;
}

__device__ Best block_best(Best b) {
    __shared__ float sv[16];
    __shared__ int32_t si[16];
    for (int off = 32; off >= 1; off >>= 1) {
        Best o;
        o.v = __shfl_xor(b.v, off, 64);
        o.i = __shfl_xor(b.i, off, 64);
        b = better(b, o);
    }
    const int wave = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
    if ((threadIdx.x & 63) == 0) { sv[wave] = b.v; si[wave] = b.i; }
    __syncthreads();
    if (threadIdx.x == 0) {
        Best r{0.0f, -1};
        for (int w = 0; w < nw; w++) r = better(r, Best{sv[w], si[w]});
        sv[0] = r.v;
        si[0] = r.i;
    }
    __syncthreads();
    return Best{sv[0], si[0]};
}

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

__global__ __launch_bounds__(64) void k_argmax_final(const float *__restrict__ x, int64_t ldx,
                                                     int nparts, const float *__restrict__ pv,
                                                     const int32_t *__restrict__ pi,
                                                     int32_t *__restrict__ idx) {
    const int64_t row = blockIdx.x;
    Best b{0.0f, -1};
    for (int j = threadIdx.x; j < nparts; j += 64) b = better(b, Best{pv[row * nparts + j], pi[row * nparts + j]});
    for (int off = 32; off >= 1; off >>= 1) {
        Best o;
        o.v = __shfl_xor(b.v, off, 64);
        o.i = __shfl_xor(b.i, off, 64);
        b = better(b, o);
    }
    if (threadIdx.x == 0) {
        float x0 = x[row * ldx];
        idx[row] = (x0 != x0 || b.i < 0) ? 0 : b.i;
    }
}

size_t argmax_scratch_bytes(int64_t rows, int64_t V) {
    int64_t parts = argmax_parts(V);
    return (size_t)rows * parts * 8 + 256;
}

int64_t argmax_parts(int64_t V) {
    int64_t p = (V + 4095) / 4096;
    if (p < 1) p = 1;
    if (p > 64) p = 64;
    return p;
}

int32_t launch_argmax(ut_ctx *ctx, const float *x, int64_t rows, int64_t V, int64_t ldx,
                      int32_t *idx, void *scratch) {
    if (rows <= 0) return UT_OK;
    const int64_t parts = argmax_parts(V);
    const int64_t chunk = (V + parts - 1) / parts;
    float *pv = (float *)scratch;
    int32_t *pi = (int32_t *)((char *)scratch + ((rows * parts * 4 + 255) & ~int64_t(255)));
    int tok = timing_begin(ctx, "argmax");
    hipLaunchKernelGGL(k_argmax_partial, dim3((unsigned)parts, (unsigned)rows), dim3(256), 0,
                       ctx->stream, x, V, ldx, chunk, pv, pi);
    UT_TRY(launch_check(ctx, "k_argmax_partial"));
    hipLaunchKernelGGL(k_argmax_final, dim3((unsigned)rows), dim3(64), 0, ctx->stream, x, ldx,
                       (int)parts, pv, pi, idx);
    timing_end(ctx, tok);
    return launch_check(ctx, "k_argmax_final");
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
