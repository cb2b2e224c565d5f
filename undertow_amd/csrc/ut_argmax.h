// ut_argmax.h -- the greedy argmax's candidate order (undertow-core/src/
// sample.rs:353-361), shared by the argmax kernels and the GEMV epilogues
// that leave per-workgroup argmax partials.
//
// A candidate is (value, index); NaN values never become candidates.  The
// better of two is the larger value, and of equal values the lower index,
// so any grouping of the candidates reduces to the same winner: the first
// index of the maximum.  The caller applies the row rule for a NaN at
// index 0 (no `x > NaN` compare succeeds, so the reference returns 0).
#pragma once

#include "ut_internal.h"

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

// The workgroup's best candidate, returned to every thread (two barriers).
__device__ inline Best block_best(Best b) {
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
    Best r{0.0f, -1};
    for (int w = 0; w < nw; w++) r = better(r, Best{sv[w], si[w]});
    __syncthreads();
    return r;
}

// Writes this workgroup's partial for each activation row from the
// per-thread candidates bm (every thread of the workgroup calls it).
template <int M>
__device__ __forceinline__ void argmax_parts_store(const ArgmaxParts &p, const Best (&bm)[M],
                                                   int64_t j) {
#pragma unroll
    for (int m = 0; m < M; m++) {
        const Best b = block_best(bm[m]);
        if (threadIdx.x == 0) {
            p.v[m * p.stride + j] = b.v;
            p.i[m * p.stride + j] = b.i;
        }
    }
}

// A candidate from one finished output value (NaN is never one).
__device__ __forceinline__ void argmax_offer(Best &b, float v, int64_t row) {
    if (v == v) b = better(b, Best{v, (int32_t)row});
}

}  // namespace ut
