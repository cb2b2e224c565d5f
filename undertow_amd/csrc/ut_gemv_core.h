// ut_gemv_core.h -- device core of the quantized skinny GEMV on gfx950.
//
// Work split of one 256-thread workgroup (4 waves of 64 lanes):
//   lane l of a wave: row group g = l >> 4 (0..3), sub-lane s = l & 15.
//   Each lane owns R = 4 weight rows (caller-chosen row pointers) and walks
//   K in steps; per step the 16 sub-lanes of a row group read 16
//   consecutive 16-byte pieces of each of its rows (a 256-byte coalesced
//   run per row per load instruction: 128-bit nibble / byte / float loads).
//   Activations for a K chunk are staged once per workgroup in LDS and read
//   back with 128-bit LDS loads, each reused across the lane's 4 rows.
//
// Arithmetic:
//   int4: v_dot8c_i32_i4 of the raw weight word (8 signed nibbles, low
//         nibble = even column, exactly the checkpoint's packing) with one
//         word of balanced base-16 activation digits; 6 digit planes.
//   int8: v_dot4c_i32_i8 of 4 weight bytes with base-256 digits; 3 planes.
//   The per-plane int32 sums are exact; the lane total
//   S = sum_p acc_p * base^p is formed in int64 and summed across the 16
//   sub-lanes exactly.  The weights are never dequantized to floats: the
//   per-row scale is applied once, out = fl(fl(S * 2^e) * scale[row]),
//   the same formula for every tiling, row count and reduction order.
//   f32:  fused multiply-add in a fixed order per lane, then a fixed
//         butterfly; the value for (row slot r, activation row m) is always
//         read from sub-lane 4*r + m, so it does not depend on M.
#pragma once

#include "ut_internal.h"

namespace ut {

constexpr int kGemvThreads = 256;
constexpr int kGemvRows = 4;         // weight rows per lane
constexpr int kLdsWords = 6144;      // 24 KiB of staged activations per WG

template <int FMT> struct FmtTraits;
template <> struct FmtTraits<UT_FMT_INT4> {
    static constexpr int kPlanes = 6;       // digit planes of x~
    static constexpr int kColsPerWord = 8;  // columns per 32-bit digit word
    static constexpr int kStepCols = 512;   // 16 lanes x 32 columns
    static constexpr int kBytesPerCol2 = 1; // 2 * bytes per column
};
template <> struct FmtTraits<UT_FMT_INT8> {
    static constexpr int kPlanes = 3;
    static constexpr int kColsPerWord = 4;
    static constexpr int kStepCols = 256;   // 16 lanes x 16 columns
    static constexpr int kBytesPerCol2 = 2;
};
template <> struct FmtTraits<UT_FMT_F32> {
    static constexpr int kPlanes = 1;       // the f32 value itself
    static constexpr int kColsPerWord = 1;
    static constexpr int kStepCols = 64;    // 16 lanes x 4 columns
    static constexpr int kBytesPerCol2 = 8;
};

// Weight steps in flight per lane (the software-pipeline depth of
// gemv_core): two for one activation row; more rows keep one, since their
// accumulators leave no registers for a second step (measured on the
// expert and dense shapes).  UT_GEMV_DEPTH overrides it for experiments.
template <int M> __host__ __device__ constexpr int gemv_depth() {
#ifdef UT_GEMV_DEPTH
    return UT_GEMV_DEPTH;
#else
    return M == 1 ? 2 : 1;
#endif
}

// Columns of one staged chunk: as many as fit kLdsWords for M rows, or at
// most CAP (> 0) when the caller's K is known to be short (fewer staging
// registers per thread).
template <int FMT, int M, int CAP = 0>
__host__ __device__ constexpr int gemv_chunk_cols() {
    using T = FmtTraits<FMT>;
    // words per column per row = planes / cols_per_word
    int cols = kLdsWords * T::kColsPerWord / (M * T::kPlanes);
    if (CAP > 0 && CAP < cols) cols = CAP;
    return cols / T::kStepCols * T::kStepCols;
}

// Activations of one GEMV: digits (int formats) or f32 values.  For int
// formats with dig == nullptr, xf is digitised while it is staged, with
// x~ = rint(x * 2^sh[m]) (sh[m] = 22 - E of the row; INT32_MIN: non-finite).
struct XSrc {
    const uint32_t *dig;  // [M][planes][KW] words (int formats)
    int64_t KW;           // words per plane row
    const float *xf;      // [M][ldx] (f32)
    int64_t ldx;
    int32_t sh[4];        // staging-time digitisation shifts (dig == nullptr)
    // dig == nullptr: the shifts come from the staged rows' own max|x|
    // (single-chunk staging only) instead of sh
    int self_max = 0;
    // bf16 activations [M][ldx] in place of xf (digitise-while-staging path
    // only): widened to f32 exactly as they are staged
    const uint16_t *xh = nullptr;
    // gemv_core<..., NORM = true> (int formats, one whole chunk from column
    // 0): each row of xf is rms-normalised with these weights (eps neps)
    // while staged, by the row digitiser's rule and reduction order, and the
    // normalised row is digitised with its own exponent (reported through
    // prep)
    const float *nw = nullptr;
    float neps = 0.0f;
};

typedef unsigned int ut_u32x4 __attribute__((ext_vector_type(4)));
template <int M>
__device__ __forceinline__ void rowmax_reduce(const ut_u32x4 (&q)[M], int32_t (&sh)[M],
                                              uint32_t *red);

// Balanced digits of 8 (int4) or 4 (int8) columns, one word per plane.
// With u = x~ + 0x888888 (int4; 0x808080 for int8) every digit of u is the
// balanced digit plus 8 (128), so the balanced digit's two's-complement
// field is the plain field of u with its top bit flipped: one add per
// column, then a shift / mask per plane.
template <int FMT>
__device__ __forceinline__ void digit_words(const float *v, int n, int32_t sh,
                                            uint32_t *w /* [planes] */) {
    constexpr int PL = FMT == UT_FMT_INT4 ? 6 : 3;
    constexpr int B = FMT == UT_FMT_INT4 ? 4 : 8;
    constexpr uint32_t OFF = FMT == UT_FMT_INT4 ? 0x888888u : 0x808080u;
    constexpr uint32_t MASK = (1u << B) - 1;
    constexpr uint32_t FLIP = FMT == UT_FMT_INT4 ? 0x88888888u : 0x80808080u;
    constexpr int KN = 32 / B;  // columns per full word
    if (n == KN) {
        // a full word: the planes are the transpose of the KN x KN matrix of
        // B-bit fields (row j = u of column j, field p = digit p), built by
        // swapping off-diagonal blocks of 1, 2 and 4 fields (int8: 1 and 2)
        uint32_t u[KN];
        if (sh >= -126 && sh <= 127) {
            // |x * 2^sh| <= 2^22, so x * 2^sh + 1.5 * 2^23 (one rounding, to
            // nearest even) lies in [2^23, 2^24], where the ulp is 1: its
            // bits are those of 1.5 * 2^23 plus rint(x * 2^sh)
            const float scale = __uint_as_float((uint32_t)(sh + 127) << 23);
#pragma unroll
            for (int j = 0; j < KN; j++)
                u[j] = __float_as_uint(__builtin_fmaf(v[j], scale, 12582912.0f)) +
                       (OFF - 0x4B400000u);
        } else {
#pragma unroll
            for (int j = 0; j < KN; j++) {
                const int32_t q = sh == INT32_MIN ? 0 : (int32_t)rintf(ldexpf(v[j], sh));
                u[j] = (uint32_t)q + OFF;
            }
        }
        auto swap_blocks = [&](int i, int k, uint32_t m, int s) {
            const uint32_t a = u[i], b = u[k];
            u[i] = (a & m) | ((b << s) & ~m);
            u[k] = ((a >> s) & m) | (b & ~m);
        };
        if constexpr (FMT == UT_FMT_INT4) {
#pragma unroll
            for (int i = 0; i < 8; i += 2) swap_blocks(i, i + 1, 0x0F0F0F0Fu, 4);
            swap_blocks(0, 2, 0x00FF00FFu, 8);
            swap_blocks(1, 3, 0x00FF00FFu, 8);
            swap_blocks(4, 6, 0x00FF00FFu, 8);
            swap_blocks(5, 7, 0x00FF00FFu, 8);
#pragma unroll
            for (int i = 0; i < 4; i++) swap_blocks(i, i + 4, 0x0000FFFFu, 16);
        } else {
            swap_blocks(0, 1, 0x00FF00FFu, 8);
            swap_blocks(2, 3, 0x00FF00FFu, 8);
            swap_blocks(0, 2, 0x0000FFFFu, 16);
            swap_blocks(1, 3, 0x0000FFFFu, 16);
        }
#pragma unroll
        for (int p = 0; p < PL; p++) w[p] = u[p] ^ FLIP;
        return;
    }
#pragma unroll
    for (int p = 0; p < PL; p++) w[p] = 0;
#pragma unroll
    for (int j = 0; j < n; j++) {
        const int32_t q = sh == INT32_MIN ? 0 : (int32_t)rintf(ldexpf(v[j], sh));
        const uint32_t u = (uint32_t)q + OFF;
#pragma unroll
        for (int p = 0; p < PL; p++) w[p] |= ((u >> (B * p)) & MASK) << (B * j);
    }
#pragma unroll
    for (int p = 0; p < PL; p++) w[p] ^= FLIP & (n * B >= 32 ? 0xffffffffu : ((1u << (n * B)) - 1));
}

// Loads through global-address-space pointers: the row pointers come from
// device-side expert tables, so the compiler cannot infer their address
// space and would otherwise emit flat loads (which also hold the LDS
// counter and force conservative waits).
// (Loaded as native vectors: a class type's copy constructor would take the
// address back to the generic space.)
typedef float ut_f32x4 __attribute__((ext_vector_type(4)));
template <typename T> __device__ __forceinline__ T ld_global(const void *p);
template <> __device__ __forceinline__ uint4 ld_global<uint4>(const void *p) {
    const ut_u32x4 v = *(const __attribute__((address_space(1))) ut_u32x4 *)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
// Streamed weights (read once per pass): non-temporal loads.
#ifndef UT_WEIGHT_NT
#define UT_WEIGHT_NT 1
#endif
__device__ __forceinline__ uint4 ld_weights(const void *p) {
#if UT_WEIGHT_NT
    const ut_u32x4 v = __builtin_nontemporal_load((const __attribute__((address_space(1))) ut_u32x4 *)p);
#else
    const ut_u32x4 v = *(const __attribute__((address_space(1))) ut_u32x4 *)p;
#endif
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float ld_global_f32(const float *p) {
    return *(const __attribute__((address_space(1))) float *)p;
}
template <> __device__ __forceinline__ float4 ld_global<float4>(const void *p) {
    const ut_f32x4 v = *(const __attribute__((address_space(1))) ut_f32x4 *)p;
    return make_float4(v.x, v.y, v.z, v.w);
}
typedef unsigned int ut_u32x2 __attribute__((ext_vector_type(2)));
template <> __device__ __forceinline__ uint2 ld_global<uint2>(const void *p) {
    const ut_u32x2 v = *(const __attribute__((address_space(1))) ut_u32x2 *)p;
    return make_uint2(v.x, v.y);
}

__device__ inline int64_t shfl_xor_i64(int64_t v, int off) {
    int lo = __shfl_xor((int)(uint32_t)(uint64_t)v, off, 16);
    int hi = __shfl_xor((int)(uint32_t)((uint64_t)v >> 32), off, 16);
    return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint64_t)(uint32_t)lo);
}

// Result of the core for lane (g, s): the totals of every (r, m), identical
// on all 16 sub-lanes for int formats; for f32 read them from sub-lane 4r+m.
template <int FMT, int M, int R = kGemvRows> struct CoreOut {
    int64_t S[R][M];
    float F[R][M];
};

// The pieces of the GEMV lane work, shared by the tiled kernels and the
// streaming expert kernel:
//   gemv_stage    stages columns [kc, kc+kcn) of the activations in LDS
//                 (whole workgroup; barriers on both sides);
//   GemvAcc       per-lane accumulators: compute() takes one step of R
//                 weight rows (16 bytes each) against the staged chunk,
//                 finish() reduces across the 16 sub-lanes of the row group.
template <int FMT, int M, int KC = gemv_chunk_cols<FMT, M>()>
__device__ __forceinline__ void gemv_stage(const XSrc &x, uint32_t *lds, int64_t kc, int kcn) {
    using T = FmtTraits<FMT>;
    constexpr int PL = T::kPlanes;
    constexpr int LW = KC / T::kColsPerWord;  // LDS words per plane row
    const int tid = threadIdx.x;
    __syncthreads();
    if constexpr (FMT == UT_FMT_F32) {
        const int n4 = kcn / 4;  // float4 per row
        for (int i = tid; i < M * n4; i += kGemvThreads) {
            int m = i / n4, c = i - m * n4;
            float4 v = ld_global<float4>(x.xf + m * x.ldx + kc + 4 * c);
            *(float4 *)(lds + m * KC + 4 * c) = v;
        }
    } else if (x.dig) {
        const int n4 = kcn / T::kColsPerWord / 4;  // uint4 per plane row
        const int64_t w0 = kc / T::kColsPerWord;
        for (int i = tid; i < M * PL * n4; i += kGemvThreads) {
            int mp = i / n4, c = i - mp * n4;
            uint4 v = ld_global<uint4>(x.dig + (int64_t)mp * x.KW + w0 + 4 * c);
            *(uint4 *)(lds + mp * LW + 4 * c) = v;
        }
    } else {
        // digitise f32 activations into the LDS planes
        constexpr int CPW = T::kColsPerWord;
        const int ng = kcn / CPW;  // words per plane row in the chunk
        for (int i = tid; i < M * ng; i += kGemvThreads) {
            const int m = i / ng, g = i - m * ng;
            const float *src = x.xf + m * x.ldx + kc + g * CPW;
            float v[CPW];
            if constexpr (CPW == 8) {
                const float4 a = ld_global<float4>(src), b = ld_global<float4>(src + 4);
                v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
                v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
            } else {
                const float4 a = ld_global<float4>(src);
                v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            }
            uint32_t w[PL];
            // select among opaque copies, not index: a runtime index into
            // x.sh (which the compiler rebuilds from a plain select chain)
            // would move the argument struct to scratch memory
            int32_t s0 = x.sh[0], s1 = x.sh[1], s2 = x.sh[2], s3 = x.sh[3];
            asm volatile("" : "+v"(s0), "+v"(s1), "+v"(s2), "+v"(s3));
            const int32_t shm = m == 0 ? s0 : m == 1 ? s1 : m == 2 ? s2 : s3;
            digit_words<FMT>(v, CPW, shm, w);
#pragma unroll
            for (int p = 0; p < PL; p++) lds[(m * PL + p) * LW + g] = w[p];
        }
    }
    __syncthreads();
}

// gemv_stage for a range that is one whole chunk, split around `issue`:
// every thread first loads its share of the chunk into registers
// (unconditionally, from a clamped index, so the wait counts stay exact),
// then `issue()` starts the caller's first weight loads, then the shares
// go to LDS.  The activation loads (L2 hits) are older than the weight
// loads, so the LDS writes wait for them alone and the weights stay in
// flight across the barrier.
// The digitise branch calls prep(sh) after issue() and before the
// barrier: a caller whose digitisation shifts are still being reduced
// finishes them there, with the weights already in flight.
struct NoPrep {
    __device__ void operator()(int32_t (&)[4]) const {}
};
struct NoMid {
    __device__ void operator()() const {}
};

template <typename T, typename Op> __device__ __forceinline__ T wave_reduce_dpp(T v, Op op);

// The normalising branch of gemv_stage_once (NORM: M <= 4 rows of x.xf,
// row stride x.ldx): thread t holds the 8-column groups t + 256 j of each
// row.  Each row's mean of squares is taken in the row digitiser's order
// (rowdig_body with one group per thread): each group's squares summed in
// f64 in column order, the groups of a 64-lane wave by the DPP butterfly,
// the wave sums in wave order (group c is lane c % 64 of wave c / 64 there,
// and lane t % 64 of wave t / 64 + 4j here, so the sums are the same), then
// r = 1/sqrt((float)(sum / K) + eps), v = (x * r) * w, the row's exponent
// from max|v|, and v's digit words into the LDS planes.  sh: the shifts.
template <int FMT, int M, int KC, typename Issue>
__device__ __forceinline__ void gemv_stage_norm(const XSrc &x, uint32_t *lds, int kcn,
                                                Issue &&issue, int32_t (&sh)[4]) {
    using T = FmtTraits<FMT>;
    constexpr int PL = T::kPlanes;
    constexpr int LW = KC / T::kColsPerWord;
    constexpr int GMAX = (KC / 8 + kGemvThreads - 1) / kGemvThreads;
    static_assert(4 * GMAX <= 16, "at most 16 virtual waves");
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int NG = kcn / 8;
    float v[M][GMAX][8], wv[GMAX][8];
#pragma unroll
    for (int j = 0; j < GMAX; j++) {
        const int c = tid + j * kGemvThreads, cc = c < NG ? c : NG - 1;
        const bool in = c < NG;
#pragma unroll
        for (int m = 0; m < M; m++) {
            const float *xr = x.xf + m * x.ldx + 8 * cc;
            const float4 a = ld_global<float4>(xr), b = ld_global<float4>(xr + 4);
            v[m][j][0] = in ? a.x : 0.0f; v[m][j][1] = in ? a.y : 0.0f;
            v[m][j][2] = in ? a.z : 0.0f; v[m][j][3] = in ? a.w : 0.0f;
            v[m][j][4] = in ? b.x : 0.0f; v[m][j][5] = in ? b.y : 0.0f;
            v[m][j][6] = in ? b.z : 0.0f; v[m][j][7] = in ? b.w : 0.0f;
        }
        const float4 p = ld_global<float4>(x.nw + 8 * cc), q = ld_global<float4>(x.nw + 8 * cc + 4);
        wv[j][0] = p.x; wv[j][1] = p.y; wv[j][2] = p.z; wv[j][3] = p.w;
        wv[j][4] = q.x; wv[j][5] = q.y; wv[j][6] = q.z; wv[j][7] = q.w;
    }
    issue();
    __builtin_amdgcn_sched_barrier(0);
    __shared__ double redd[M][16];
    __shared__ uint32_t redu[M][4];
#pragma unroll
    for (int m = 0; m < M; m++)
#pragma unroll
        for (int j = 0; j < GMAX; j++) {
            double acc = 0.0;
#pragma unroll
            for (int q = 0; q < 8; q++) acc += (double)v[m][j][q] * (double)v[m][j][q];
            acc = wave_reduce_dpp(acc, [](double p, double q) { return p + q; });
            if (lane == 0) redd[m][wave + 4 * j] = acc;
        }
    for (int i = tid; i < M * 16; i += kGemvThreads)
        if (i % 16 >= 4 * GMAX) redd[i / 16][i % 16] = 0.0;
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
    for (int m = 0; m < M; m++) {
        double ss = redd[m][0];
        for (int i = 1; i < 16; i++) ss += redd[m][i];
        const float r = 1.0f / sqrtf(__fadd_rn((float)(ss / (double)kcn), x.neps));
        uint32_t mx = 0;
#pragma unroll
        for (int j = 0; j < GMAX; j++) {
            const bool in = tid + j * kGemvThreads < NG;
#pragma unroll
            for (int q = 0; q < 8; q++) {
                v[m][j][q] = __fmul_rn(__fmul_rn(v[m][j][q], r), wv[j][q]);
                if (in) mx = max(mx, __float_as_uint(fabsf(v[m][j][q])));
            }
        }
        mx = wave_reduce_dpp(mx, [](uint32_t p, uint32_t q) { return p > q ? p : q; });
        if (lane == 0) redu[m][wave] = mx;
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
    for (int m = 0; m < M; m++) {
        const uint32_t mx = max(max(redu[m][0], redu[m][1]), max(redu[m][2], redu[m][3]));
        const bool bad = mx >= 0x7f800000u;
        int E = 0;
        if (!bad && mx != 0) (void)frexpf(__uint_as_float(mx), &E);
        sh[m] = bad ? INT32_MIN : 22 - E;
#pragma unroll
        for (int j = 0; j < GMAX; j++) {
            const int c = tid + j * kGemvThreads;
            if (c >= NG) continue;
            if constexpr (FMT == UT_FMT_INT4) {
                uint32_t w[PL];
                digit_words<UT_FMT_INT4>(v[m][j], 8, sh[m], w);
#pragma unroll
                for (int p = 0; p < PL; p++) lds[(m * PL + p) * LW + c] = w[p];
            } else {
                uint32_t w[PL], w2[PL];
                digit_words<UT_FMT_INT8>(v[m][j], 4, sh[m], w);
                digit_words<UT_FMT_INT8>(v[m][j] + 4, 4, sh[m], w2);
#pragma unroll
                for (int p = 0; p < PL; p++)
                    *(uint2 *)(lds + (m * PL + p) * LW + 2 * c) = make_uint2(w[p], w2[p]);
            }
        }
    }
}

template <int FMT, int M, int KC, bool NORM = false, typename Issue, typename Prep = NoPrep>
__device__ __forceinline__ void gemv_stage_once(const XSrc &x, uint32_t *lds, int64_t kc, int kcn,
                                                Issue &&issue, Prep &&prep = Prep{}) {
    using T = FmtTraits<FMT>;
    constexpr int PL = T::kPlanes;
    constexpr int CPW = T::kColsPerWord;
    constexpr int LW = KC / CPW;
    const int tid = threadIdx.x;
    // a separate instantiation: its registers would lower every other
    // kernel's occupancy
    if constexpr (NORM) {
        static_assert(FMT != UT_FMT_F32, "normalising staging: int formats");
        int32_t shl[4] = {0, 0, 0, 0};
        gemv_stage_norm<FMT, M, KC>(x, lds, kcn, issue, shl);
        prep(shl);
        __syncthreads();
        return;
    }
    if constexpr (FMT == UT_FMT_F32) {
        constexpr int NI = (M * (KC / 4) + kGemvThreads - 1) / kGemvThreads;
        const int n4 = kcn / 4, tot = M * n4;
        float4 v[NI];
#pragma unroll
        for (int j = 0; j < NI; j++) {
            const int i = tid + j * kGemvThreads, ic = i < tot ? i : tot - 1;
            const int m = ic / n4, c = ic - m * n4;
            v[j] = ld_global<float4>(x.xf + m * x.ldx + kc + 4 * c);
        }
        issue();
        __syncthreads();
#pragma unroll
        for (int j = 0; j < NI; j++) {
            const int i = tid + j * kGemvThreads;
            if (i < tot) {
                const int m = i / n4, c = i - m * n4;
                *(float4 *)(lds + m * KC + 4 * c) = v[j];
            }
        }
    } else if (x.dig) {
        constexpr int NI = (M * PL * (LW / 4) + kGemvThreads - 1) / kGemvThreads;
        const int n4 = kcn / CPW / 4, tot = M * PL * n4;
        const int64_t w0 = kc / CPW;
        uint4 v[NI];
#pragma unroll
        for (int j = 0; j < NI; j++) {
            const int i = tid + j * kGemvThreads, ic = i < tot ? i : tot - 1;
            const int mp = ic / n4, c = ic - mp * n4;
            v[j] = ld_global<uint4>(x.dig + (int64_t)mp * x.KW + w0 + 4 * c);
        }
        issue();
        __syncthreads();
#pragma unroll
        for (int j = 0; j < NI; j++) {
            const int i = tid + j * kGemvThreads;
            if (i < tot) {
                const int mp = i / n4, c = i - mp * n4;
                *(uint4 *)(lds + mp * LW + 4 * c) = v[j];
            }
        }
    } else {
        // digitise f32 activations into the LDS planes
        constexpr int NI = (M * LW + kGemvThreads - 1) / kGemvThreads;
        constexpr int NV = CPW / 4;  // float4 per word group
        const int ng = kcn / CPW, tot = M * ng;
        float4 v[NI][NV];
#pragma unroll
        for (int j = 0; j < NI; j++) {
            const int i = tid + j * kGemvThreads, ic = i < tot ? i : tot - 1;
            const int m = ic / ng, g = ic - m * ng;
            if (x.xh) {
                const uint16_t *hs = x.xh + m * x.ldx + kc + g * CPW;
#pragma unroll
                for (int q = 0; q < NV; q++) {
                    // little-endian pairs: the low half is the even value
                    const uint2 hv = ld_global<uint2>(hs + 4 * q);
                    v[j][q] = make_float4(__uint_as_float(hv.x << 16),
                                          __uint_as_float(hv.x & 0xffff0000u),
                                          __uint_as_float(hv.y << 16),
                                          __uint_as_float(hv.y & 0xffff0000u));
                }
            } else {
                const float *src = x.xf + m * x.ldx + kc + g * CPW;
#pragma unroll
                for (int q = 0; q < NV; q++) v[j][q] = ld_global<float4>(src + 4 * q);
            }
        }
        issue();
        // prep's waits stay behind every load above
        __builtin_amdgcn_sched_barrier(0);
        int32_t shl[4] = {x.sh[0], x.sh[1], x.sh[2], x.sh[3]};
        if (x.self_max) {
            // max|x| of each row over the whole staged range (kcn = the
            // row's columns): the row digitiser's exponent rule
            ut_u32x4 q[M];
#pragma unroll
            for (int m = 0; m < M; m++) q[m] = ut_u32x4{0u, 0u, 0u, 0u};
#pragma unroll
            for (int j = 0; j < NI; j++) {
                const int i = tid + j * kGemvThreads;
                const int mi = i < tot ? i / ng : -1;
                uint32_t b = 0;
#pragma unroll
                for (int q4 = 0; q4 < NV; q4++) {
                    b = max(b, max(max(__float_as_uint(fabsf(v[j][q4].x)), __float_as_uint(fabsf(v[j][q4].y))),
                                   max(__float_as_uint(fabsf(v[j][q4].z)), __float_as_uint(fabsf(v[j][q4].w)))));
                }
#pragma unroll
                for (int m = 0; m < M; m++)
                    if (mi == m) q[m][0] = max(q[m][0], b);
            }
            __shared__ uint32_t red[4 * M];
            int32_t sh[M];
            rowmax_reduce<M>(q, sh, red);
#pragma unroll
            for (int m = 0; m < M; m++) shl[m] = sh[m];
        }
        prep(shl);
        __syncthreads();
#pragma unroll
        for (int j = 0; j < NI; j++) {
            const int i = tid + j * kGemvThreads;
            if (i < tot) {
                const int m = i / ng, g = i - m * ng;
                float f[CPW];
#pragma unroll
                for (int q = 0; q < NV; q++) {
                    f[4 * q] = v[j][q].x; f[4 * q + 1] = v[j][q].y;
                    f[4 * q + 2] = v[j][q].z; f[4 * q + 3] = v[j][q].w;
                }
                uint32_t w[PL];
                const int32_t shm = m == 0 ? shl[0] : m == 1 ? shl[1] : m == 2 ? shl[2] : shl[3];
                digit_words<FMT>(f, CPW, shm, w);
#pragma unroll
                for (int p = 0; p < PL; p++) lds[(m * PL + p) * LW + g] = w[p];
            }
        }
    }
    __syncthreads();
}

template <int FMT, int M, int R, int KC_ = gemv_chunk_cols<FMT, M>()> struct GemvAcc {
    using T = FmtTraits<FMT>;
    static constexpr int KC = KC_;
    static constexpr int PL = T::kPlanes;
    static constexpr int LW = KC / T::kColsPerWord;
    int32_t acc[R][M][PL];
    float facc[R][M];

    __device__ __forceinline__ void zero() {
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int m = 0; m < M; m++) {
                facc[r][m] = 0.0f;
#pragma unroll
                for (int p = 0; p < PL; p++) acc[r][m][p] = 0;
            }
    }

    // c0: this lane's first column within the staged chunk
    __device__ __forceinline__ void compute(const uint32_t *lds, const uint4 (&wv)[R], int c0) {
        if constexpr (FMT == UT_FMT_F32) {
#pragma unroll
            for (int m = 0; m < M; m++) {
                const float4 xv = *(const float4 *)(lds + m * KC + c0);
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const float4 wf = *(const float4 *)&wv[r];
                    float a = facc[r][m];
                    a = __builtin_fmaf(wf.x, xv.x, a);
                    a = __builtin_fmaf(wf.y, xv.y, a);
                    a = __builtin_fmaf(wf.z, xv.z, a);
                    a = __builtin_fmaf(wf.w, xv.w, a);
                    facc[r][m] = a;
                }
            }
        } else {
            const int wc = c0 / T::kColsPerWord;  // first word of this lane's columns
#pragma unroll
            for (int m = 0; m < M; m++) {
#pragma unroll
                for (int p = 0; p < PL; p++) {
                    const uint4 xv = *(const uint4 *)(lds + (m * PL + p) * LW + wc);
#pragma unroll
                    for (int r = 0; r < R; r++) {
                        int a = acc[r][m][p];
                        if constexpr (FMT == UT_FMT_INT4) {
                            a = __builtin_amdgcn_sdot8((int)wv[r].x, (int)xv.x, a, false);
                            a = __builtin_amdgcn_sdot8((int)wv[r].y, (int)xv.y, a, false);
                            a = __builtin_amdgcn_sdot8((int)wv[r].z, (int)xv.z, a, false);
                            a = __builtin_amdgcn_sdot8((int)wv[r].w, (int)xv.w, a, false);
                        } else {
                            a = __builtin_amdgcn_sdot4((int)wv[r].x, (int)xv.x, a, false);
                            a = __builtin_amdgcn_sdot4((int)wv[r].y, (int)xv.y, a, false);
                            a = __builtin_amdgcn_sdot4((int)wv[r].z, (int)xv.z, a, false);
                            a = __builtin_amdgcn_sdot4((int)wv[r].w, (int)xv.w, a, false);
                        }
                        acc[r][m][p] = a;
                    }
                }
            }
        }
    }

    // reduce across the 16 sub-lanes of the row group
    __device__ __forceinline__ void finish(CoreOut<FMT, M, R> &res) const {
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int m = 0; m < M; m++) {
                if constexpr (FMT == UT_FMT_F32) {
                    float v = facc[r][m];
#pragma unroll
                    for (int off = 8; off >= 1; off >>= 1) v += __shfl_xor(v, off, 16);
                    res.F[r][m] = v;
                    res.S[r][m] = 0;
                } else {
                    constexpr int SH = FMT == UT_FMT_INT4 ? 4 : 8;
                    int64_t t = 0;
#pragma unroll
                    for (int p = PL - 1; p >= 0; p--) t = t * (1 << SH) + (int64_t)acc[r][m][p];
#pragma unroll
                    for (int off = 8; off >= 1; off >>= 1) t += shfl_xor_i64(t, off);
                    res.S[r][m] = t;
                    res.F[r][m] = 0.0f;
                }
            }
    }
};

// One step of R weight rows for this lane (16 bytes each, at column col).
template <int FMT, int R>
__device__ __forceinline__ void gemv_load(const uint8_t *const rows[R], int64_t col, uint4 (&w)[R]) {
    const int64_t boff = col * FmtTraits<FMT>::kBytesPerCol2 / 2;
#pragma unroll
    for (int r = 0; r < R; r++) w[r] = ld_weights(rows[r] + boff);
}

// rows[r]: byte pointer of row r (already clamped to a valid row).
// K: columns (the caller's contract: int4 K % 32 == 0, int8 K % 16 == 0,
// f32 K % 4 == 0, rows 16-byte aligned).
//
// The K loop is software-pipelined DEPTH steps deep: the weights of the
// next DEPTH-1 steps are in flight while a step computes, and the first
// loads are issued before the first activation chunk is staged, so the LDS
// barrier does not drain the memory pipe.
//
// When the whole column range is one LDS chunk of whole steps (the expert
// and most dense shapes) the activations are staged once and the loop has
// no staging branch and no per-lane bounds: straight-line code in which
// the compiler's wait counts keep the DEPTH-1 younger steps in flight (a
// staging branch inside the loop makes it drain every load first).
// Whether gemv_core stages the columns [k_begin, kend) once (the
// straight-line path, the only one that calls prep).
template <int FMT, int M, int KC = gemv_chunk_cols<FMT, M>()>
__device__ __forceinline__ bool gemv_one_chunk(int64_t k_begin, int64_t kend) {
    constexpr int STEP = FmtTraits<FMT>::kStepCols;
    return kend > k_begin && kend - k_begin <= KC && (kend - k_begin) % STEP == 0;
}

//
// prep: see gemv_stage_once (single-chunk path with f32 activations only;
// the caller must not rely on it elsewhere).  mid: runs before the first
// weight loads, which read rows[] only then (so mid may still fill rows
// in); on the single-chunk path after the activation loads are issued.
// KC: the staged chunk's columns (gemv_chunk_cols, possibly capped).
// STAGED: the caller has already staged the one chunk into LDS (and passed
// a workgroup barrier after it): straight to the weights.
template <int FMT, int M, int R = kGemvRows, int DEPTH = gemv_depth<M>(),
          int KC = gemv_chunk_cols<FMT, M>(), bool STAGED = false, typename Prep = NoPrep,
          typename Mid = NoMid, bool NORM = false>
__device__ __forceinline__ void gemv_core(const uint8_t *const rows[R], int64_t K, const XSrc &x,
                                          uint32_t *lds, CoreOut<FMT, M, R> &res,
                                          int64_t k_begin = 0, int64_t k_end = -1,
                                          Prep &&prep = Prep{}, Mid &&mid = Mid{}) {
    using T = FmtTraits<FMT>;
    constexpr int STEP = T::kStepCols;    // columns per step (16 sub-lanes)
    constexpr int LANE_COLS = STEP / 16;  // columns per lane per step
    const int s = threadIdx.x & 15;
    GemvAcc<FMT, M, R, KC> A;
    A.zero();
    // columns [k_begin, k_end) (k_begin a multiple of STEP); K bounds loads.
    const int64_t kend = k_end < 0 || k_end > K ? K : k_end;
    const int64_t nsteps = kend > k_begin ? (kend - k_begin + STEP - 1) / STEP : 0;
    const int64_t lane_col = k_begin + (int64_t)s * LANE_COLS;
    uint4 wq[DEPTH][R];
    auto loadk = [&](uint4 (&w)[R], int64_t col) { if (col < kend) gemv_load<FMT, R>(rows, col, w); };
    if (gemv_one_chunk<FMT, M, KC>(k_begin, kend)) {
        // unconditional (clamped) first loads: a skipped load on any path
        // into the loop would make the wait counts inside it conservative
        auto first = [&]() {
            mid();
#pragma unroll
            for (int u = 0; u < DEPTH; u++)
                gemv_load<FMT, R>(rows, lane_col + (u < nsteps ? u : nsteps - 1) * STEP, wq[u]);
        };
        if constexpr (STAGED)
            first();
        else
            gemv_stage_once<FMT, M, KC, NORM>(x, lds, k_begin, (int)(kend - k_begin), first, prep);
        const int c0 = s * LANE_COLS;
        int64_t t = 0;
        for (; t + 2 * DEPTH <= nsteps; t += DEPTH) {
#pragma unroll
            for (int u = 0; u < DEPTH; u++) {
                A.compute(lds, wq[u], (int)((t + u) * STEP) + c0);
                gemv_load<FMT, R>(rows, lane_col + (t + u + DEPTH) * STEP, wq[u]);
                // keep the scheduler from sinking the loads below the next
                // step's compute (which would drain the pipe every DEPTH steps)
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        // the last DEPTH..2*DEPTH-1 steps (fewer when nsteps < DEPTH)
#pragma unroll
        for (int i = 0; i < 2 * DEPTH; i++) {
            if (t + i < nsteps) {
                A.compute(lds, wq[i % DEPTH], (int)((t + i) * STEP) + c0);
                if (t + i + DEPTH < nsteps)
                    gemv_load<FMT, R>(rows, lane_col + (t + i + DEPTH) * STEP, wq[i % DEPTH]);
            }
        }
        A.finish(res);
        return;
    }
    mid();
#pragma unroll
    for (int u = 0; u < DEPTH; u++) loadk(wq[u], lane_col + u * STEP);
    int64_t kc = k_begin, chunk_end = k_begin;
    for (int64_t t = 0; t < nsteps; t += DEPTH) {
#pragma unroll
        for (int u = 0; u < DEPTH; u++) {
            if (t + u < nsteps) {
                const int64_t cu = (t + u) * STEP + lane_col;
                if (k_begin + (t + u) * STEP >= chunk_end) {
                    kc = k_begin + (t + u) * STEP;
                    const int kcn = (int)((kend - kc) < KC ? (kend - kc) : KC);
                    chunk_end = kc + kcn;
                    gemv_stage<FMT, M, KC>(x, lds, kc, kcn);
                }
                if (cu < kend) A.compute(lds, wq[u], (int)(cu - kc));
                loadk(wq[u], cu + DEPTH * STEP);
            }
        }
    }
    A.finish(res);
}

template <typename T, typename Op>
__device__ __forceinline__ T block_reduce(T v, Op op, T *red4) {
    for (int off = 32; off >= 1; off >>= 1) v = op(v, __shfl_xor(v, off, 64));
    if ((threadIdx.x & 63) == 0) red4[threadIdx.x >> 6] = v;
    __syncthreads();
    T r = op(op(red4[0], red4[1]), op(red4[2], red4[3]));
    __syncthreads();
    return r;
}

// Wave reductions by DPP moves (no LDS round trips): after the quad, half-row
// and row mirror steps every lane holds its 16-lane row's value; the row
// broadcasts then fold rows 0..3 into lane 63.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t v, uint32_t identity) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)identity, (int)v, CTRL, ROW_MASK, 0xF, false);
}
template <typename T> struct DppBits;
template <> struct DppBits<uint32_t> {
    template <int C, int RM> static __device__ __forceinline__ uint32_t mov(uint32_t v) { return dpp_mov<C, RM>(v, 0u); }
    static __device__ __forceinline__ uint32_t lane63(uint32_t v) { return __builtin_amdgcn_readlane(v, 63); }
};
template <> struct DppBits<double> {
    template <int C, int RM> static __device__ __forceinline__ double mov(double v) {
        const uint64_t u = __double_as_longlong(v);
        const uint32_t lo = dpp_mov<C, RM>((uint32_t)u, 0u), hi = dpp_mov<C, RM>((uint32_t)(u >> 32), 0u);
        return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));  // identity 0.0
    }
    static __device__ __forceinline__ double lane63(double v) {
        const uint64_t u = __double_as_longlong(v);
        const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)u, 63), hi = __builtin_amdgcn_readlane((uint32_t)(u >> 32), 63);
        return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
    }
};
// identity of op must be all-zero bits (sum of doubles, max of unsigned)
template <typename T, typename Op>
__device__ __forceinline__ T wave_reduce_dpp(T v, Op op) {
    using B = DppBits<T>;
    v = op(v, B::template mov<0xB1, 0xF>(v));   // quad_perm 1,0,3,2
    v = op(v, B::template mov<0x4E, 0xF>(v));   // quad_perm 2,3,0,1
    v = op(v, B::template mov<0x141, 0xF>(v));  // row_half_mirror
    v = op(v, B::template mov<0x140, 0xF>(v));  // row_mirror
    v = op(v, B::template mov<0x142, 0xA>(v));  // row_bcast15
    v = op(v, B::template mov<0x143, 0xC>(v));  // row_bcast31
    return B::lane63(v);
}

template <> struct DppBits<float> {
    template <int C, int RM> static __device__ __forceinline__ float mov(float v) {
        return __uint_as_float(dpp_mov<C, RM>(__float_as_uint(v), 0u));
    }
    static __device__ __forceinline__ float lane63(float v) {
        return __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 63));
    }
};

// The digitisation shifts of M activation rows from partial maxima of |x|
// (float bits, nparts per row): 22 - E with max < 2^E, INT32_MIN for a
// non-finite row.  Whole workgroup of kGemvThreads; red: 4*M words of LDS.
// 16-byte loads when nparts % 4 == 0 (16-byte aligned rows), DPP wave
// maxima, LDS-only barriers.
// This thread's share of the partial maxima: rowmax_load issues the loads
// (one 16-byte load per thread per row when nparts % 4 == 0 and
// nparts <= 4 * kGemvThreads; threads past the end re-read the row's first
// four, which leaves the maximum unchanged) without waiting for them, so a
// caller can put them ahead of other loads; rowmax_reduce finishes the
// shifts.
template <int M>
__device__ __forceinline__ void rowmax_load(const uint32_t *parts, int nparts, ut_u32x4 (&q)[M]) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int m = 0; m < M; m++) {
        const uint32_t *pr = parts + (int64_t)m * nparts;
        if ((nparts & 3) == 0 && nparts <= 4 * kGemvThreads) {
            q[m] = *(const ut_u32x4 *)(pr + (4 * tid < nparts ? 4 * tid : 0));
            continue;
        }
        uint32_t v = 0;
        if ((nparts & 3) == 0) {
            for (int i = 4 * tid; i < nparts; i += 4 * kGemvThreads) {
                const ut_u32x4 w = *(const ut_u32x4 *)(pr + i);
                v = max(v, max(max(w[0], w[1]), max(w[2], w[3])));
            }
        } else {
            for (int i = tid; i < nparts; i += kGemvThreads) v = max(v, pr[i]);
        }
        q[m] = ut_u32x4{v, v, v, v};
    }
}

template <int M>
__device__ __forceinline__ void rowmax_reduce(const ut_u32x4 (&q)[M], int32_t (&sh)[M],
                                              uint32_t *red) {
    uint32_t mx[M];
    const int tid = threadIdx.x;
#pragma unroll
    for (int m = 0; m < M; m++)
        mx[m] = wave_reduce_dpp(max(max(q[m][0], q[m][1]), max(q[m][2], q[m][3])),
                                [](uint32_t p, uint32_t q) { return p > q ? p : q; });
    if ((tid & 63) == 0)
#pragma unroll
        for (int m = 0; m < M; m++) red[(tid >> 6) * M + m] = mx[m];
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
    for (int m = 0; m < M; m++) {
        const uint32_t r = max(max(red[m], red[M + m]), max(red[2 * M + m], red[3 * M + m]));
        int E = 0;
        if (r < 0x7f800000u && r != 0) (void)frexpf(__uint_as_float(r), &E);
        sh[m] = r >= 0x7f800000u ? INT32_MIN : 22 - E;
    }
    // red may be reused right away by the caller
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int M>
__device__ __forceinline__ void rowmax_shifts(const uint32_t *parts, int nparts,
                                              int32_t (&sh)[M], uint32_t *red) {
    ut_u32x4 q[M];
    rowmax_load<M>(parts, nparts, q);
    rowmax_reduce<M>(q, sh, red);
}

__device__ __forceinline__ int32_t rowmax_shift(const uint32_t *parts, int nparts, int64_t row,
                                                uint32_t *red4) {
    int32_t sh[1];
    rowmax_shifts<1>(parts + row * nparts, nparts, sh, red4);
    return sh[0];
}

// Converts an exact integer total to the reference's f32 row value:
// fl(fl(S * 2^e) * scale).  e == INT32_MIN marks a non-finite activation row.
__device__ __forceinline__ float int_total_to_f32(int64_t S, int32_t e, float scale) {
    if (e == INT32_MIN) return __int_as_float(0x7fc00000);
    float v = (float)ldexp((double)S, e);
    return __fmul_rn(v, scale);
}

// Value of (r, m) from the core result: for f32 read sub-lane 4r+m (callers
// run this on that lane), for int formats every sub-lane holds it.
template <int FMT, int M, int R>
__device__ __forceinline__ float core_value(const CoreOut<FMT, M, R> &res, int r, int m,
                                            const int32_t *exps, const float *scales,
                                            int64_t row) {
    if constexpr (FMT == UT_FMT_F32) return res.F[r][m];
    else return int_total_to_f32(res.S[r][m], exps[m], ld_global_f32(scales + row));
}

}  // namespace ut
