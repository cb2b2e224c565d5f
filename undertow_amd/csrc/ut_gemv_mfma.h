// ut_gemv_mfma.h -- int4 skinny GEMV for 2..5 activation rows on the matrix
// cores (v_mfma_i32_16x16x64_i8), the same exact-integer totals as the
// dot-product core in ut_gemv_core.h.
//
// Why: with M activation rows the dot-product core reads 6*M digit words
// from LDS and issues 24*M dot instructions per 16 weight bytes and row;
// past two rows its accumulators (6 planes x M x rows per lane) leave room
// for one weight step in flight, and the GEMV is latency-bound far below
// the HBM rate.  On the matrix core one wave computes 16 weight rows
// against N = 3*M columns (three base-256 digit planes per activation row)
// with a 4-register accumulator, so the weight pipe can be kept deep.
//
// Work split of a wave: 16 weight rows (row i = lane & 15 is the A-operand
// row this lane loads); lane group kg = lane >> 4 owns, per 128-column
// step, the 32 columns [128j + 32kg, +32): one 16-byte load of packed int4,
// unpacked to two 16-byte A operands of sign-extended bytes.  The byte
// order inside an operand is a permutation of those columns (per 8-column
// group: the even columns, then the odd ones, which is what masking the
// low and high nibbles of a packed word gives); the staged activation
// digits use the same permutation, and since A and B share the K order of
// each lane group and byte, the products pair the same columns.
//
// Activations: x~ = rint(x * 2^sh) as in the dot-product core (the same
// shift, so the same integer), written as three balanced base-256 digit
// planes; plane row n = 3m + p holds the digits of activation row m.
// Totals: S = sum_p 256^p * C[row][3m + p], exact in int64 (|C| < 2^31:
// K * 8 * 128 <= 2^31 for K <= 2^21).
#pragma once

#include "ut_gemv_core.h"

namespace ut {

typedef int ut_i32x4 __attribute__((ext_vector_type(4)));

// Staged digit row pitch: the chunk's columns plus 16 bytes, so the 16
// plane rows a lane group reads sit in distinct LDS banks.
template <int KC> __host__ __device__ constexpr int mfma_row_bytes() { return KC + 16; }
template <int M, int KC> __host__ __device__ constexpr int mfma_lds_words() {
    return 3 * M * mfma_row_bytes<KC>() / 4;
}
constexpr int kMfmaStepCols = 128;  // columns per step (4 lane groups x 32)

// Sign-extended bytes of the 4 nibbles (bits 0-3 of each byte) of t, where
// t holds each nibble with its top bit flipped: ((u ^ 8) + 120) ^ 128 is u's
// two's-complement value for a nibble u, and no byte carries.
__device__ __forceinline__ int mfma_sext4(uint32_t t) {
    return (int)(((t & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u);
}

// Stage the columns [kc, kc + kcn) (kcn <= KC, a multiple of 8) of M f32
// activation rows (row m at xf + m*ldx) as digit planes in the permuted
// column order.  issue() runs after the activation loads are issued (the
// caller's first weight loads); prep(sh) fills the per-row shifts
// (INT32_MIN: non-finite row, zero digits).
template <int M, int KC, typename Issue, typename Prep>
__device__ __forceinline__ void mfma_stage_f32(const float *xf, int64_t ldx, int64_t kc, int kcn,
                                               uint8_t *lds, Issue &&issue, Prep &&prep) {
    constexpr int NI = (M * (KC / 8) + kGemvThreads - 1) / kGemvThreads;
    constexpr int RB = mfma_row_bytes<KC>();
    const int NG = kcn / 8, TOT = M * NG;
    const int tid = threadIdx.x;
    float4 v[NI][2];
#pragma unroll
    for (int j = 0; j < NI; j++) {
        const int i = tid + j * kGemvThreads, ic = i < TOT ? i : TOT - 1;
        const int m = ic / NG, g = ic - m * NG;
        const float *src = xf + m * ldx + kc + 8 * g;
        v[j][0] = ld_global<float4>(src);
        v[j][1] = ld_global<float4>(src + 4);
    }
    issue();
    __builtin_amdgcn_sched_barrier(0);
    int32_t shl[4] = {0, 0, 0, 0};
    prep(shl);
#pragma unroll
    for (int j = 0; j < NI; j++) {
        const int i = tid + j * kGemvThreads;
        if (i < TOT) {
            const int m = i / NG, g = i - m * NG;
            const int32_t sh = m == 0 ? shl[0] : m == 1 ? shl[1] : m == 2 ? shl[2] : shl[3];
            const float ev[4] = {v[j][0].x, v[j][0].z, v[j][1].x, v[j][1].z};
            const float od[4] = {v[j][0].y, v[j][0].w, v[j][1].y, v[j][1].w};
            uint32_t we[3], wo[3];
            digit_words<UT_FMT_INT8>(ev, 4, sh, we);
            digit_words<UT_FMT_INT8>(od, 4, sh, wo);
#pragma unroll
            for (int p = 0; p < 3; p++)
                *(uint2 *)(lds + (3 * m + p) * RB + 8 * g) = make_uint2(we[p], wo[p]);
        }
    }
    __syncthreads();
}

// acc[q] = C[4kg + q][n] (lane group kg, sub-lane n): sub-lane s = 4r + m
// of group kg collects row 4kg + r's planes 3m, 3m+1, 3m+2 from sub-lanes
// 3m + p into res.S[r][m].
template <int M>
__device__ __forceinline__ void mfma_collect(const ut_i32x4 &acc, CoreOut<UT_FMT_INT4, M, 4> &res) {
    const int lane = threadIdx.x & 63, n = lane & 15;
    const int r_me = n >> 2, m_me = n & 3;
    int64_t S = 0;
#pragma unroll
    for (int q = 0; q < 4; q++) {
#pragma unroll
        for (int p = 0; p < 3; p++) {
            const int src = (lane & 48) | (3 * m_me + p);
            const int v = __shfl(acc[q], src, 64);
            if (q == r_me) S += (int64_t)v * (int64_t)(1 << (8 * p));
        }
    }
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int m = 0; m < M; m++) {
            res.S[r][m] = S;
            res.F[r][m] = 0.0f;
        }
}

// Weight loads of the int4 kernels.  The A operand gives a lane 16 bytes of
// one row (lane (i, kg): row i, bytes [64j + 16kg, +16) of step j), so
// loading it directly asks for 64 bytes of each row per instruction, half a
// 128-byte line, and every line twice.  Instead a wave loads a 16-row tile
// in 128-byte segments (two steps) as two instructions of 8 rows x 128
// contiguous bytes (lane l: tile row 8r + l/8, bytes 16 (l % 8)), writes
// them to a wave-private LDS area and reads the A operands back from it:
// whole lines per request.  Area layout: rows 2q and 2q + 1 share 256
// bytes, their 16-byte chunks XOR-swizzled by q, so the 16 rows one read
// touches cover all 64 banks.  rows[w][r]: this lane's load row of tile w,
// instruction r (tile row 8r + lane / 8), clamped to a valid row.
constexpr int kI4SegBytes = 128;                    // two 128-column steps of a row
constexpr int kI4WaveAreaBytes = 16 * kI4SegBytes;  // one segment of a 16-row tile
__device__ __forceinline__ int i4_area_off(int row, int chunk) {
    return (row >> 1) * 256 + (row & 1) * 128 + 16 * (chunk ^ ((row >> 1) & 7));
}

// Segment sg of tile w into registers (two 16-byte loads); a last segment
// holding one step (odd nsteps) re-reads the first half for its second.
template <int TW>
__device__ __forceinline__ void i4_seg_load(uint4 (&d)[TW][2], const uint8_t *const (&rows)[TW][2],
                                            int64_t kb, int sg, int nsteps) {
    const int lane = threadIdx.x & 63, c = lane & 7;
    const int nseg = (nsteps + 1) >> 1;
    const int g = sg < nseg ? sg : nseg - 1;
    const int cc = (2 * g + (c >> 2) < nsteps) ? c : c - 4;
    const int64_t off = kb + (int64_t)kI4SegBytes * g + 16 * cc;
#pragma unroll
    for (int w = 0; w < TW; w++)
#pragma unroll
        for (int r = 0; r < 2; r++) d[w][r] = ld_weights(rows[w][r] + off);
}

template <int TW>
__device__ __forceinline__ void i4_seg_store(const uint4 (&d)[TW][2], uint8_t *warea) {
    const int lane = threadIdx.x & 63, c = lane & 7;
#pragma unroll
    for (int w = 0; w < TW; w++)
#pragma unroll
        for (int r = 0; r < 2; r++)
            *(uint4 *)(warea + w * kI4WaveAreaBytes + i4_area_off(8 * r + (lane >> 3), c)) = d[w][r];
}

// The MFMA step s (0 or 1) of a staged segment for every tile: this lane's
// A bytes (row lane % 16, chunk 4s + lane / 16) unpacked to two operands.
template <int TW>
__device__ __forceinline__ void i4_seg_mfma(const uint8_t *warea, int s, const ut_i32x4 &B0,
                                            const ut_i32x4 &B1, ut_i32x4 (&acc)[TW]) {
    const int lane = threadIdx.x & 63, n = lane & 15, kg = lane >> 4;
#pragma unroll
    for (int w = 0; w < TW; w++) {
        const uint4 wv = *(const uint4 *)(warea + w * kI4WaveAreaBytes + i4_area_off(n, 4 * s + kg));
        const uint32_t X = 0x88888888u;
        const uint32_t a0 = wv.x ^ X, a1 = wv.y ^ X, a2 = wv.z ^ X, a3 = wv.w ^ X;
        const ut_i32x4 A0 = {mfma_sext4(a0), mfma_sext4(a0 >> 4), mfma_sext4(a1), mfma_sext4(a1 >> 4)};
        const ut_i32x4 A1 = {mfma_sext4(a2), mfma_sext4(a2 >> 4), mfma_sext4(a3), mfma_sext4(a3 >> 4)};
        acc[w] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, B0, acc[w], 0, 0, 0);
        acc[w] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, B1, acc[w], 0, 0, 0);
    }
}

// One wave: TW tiles of 16 rows (sharing the B operand) x M activation rows
// over the columns [0, K) staged whole (K <= KC, K % 128 == 0).  DS
// segments (two steps each) of weights in flight.  The total for (wave row
// 4g + r, activation row m) lands in res.S[r][m] of sub-lane 4r + m of
// lane group g (the dot-product core's convention with 4 rows per lane).
template <int M, int DS, int KC, int TW, typename Prep>
__device__ __forceinline__ void mfma_gemv_i4_f32x(const uint8_t *const (&rows)[TW][2], int64_t K,
                                                  const float *xf, int64_t ldx, uint8_t *lds,
                                                  uint8_t *warea,
                                                  CoreOut<UT_FMT_INT4, M, 4> (&res)[TW],
                                                  Prep &&prep) {
    static_assert(M >= 1 && M <= 4, "three digit planes per row, 16 columns");
    constexpr int RB = mfma_row_bytes<KC>();
    const int lane = threadIdx.x & 63, n = lane & 15, kg = lane >> 4;
    const int nsteps = (int)(K / kMfmaStepCols), nseg = (nsteps + 1) >> 1;
    uint4 wq[DS][TW][2];
    mfma_stage_f32<M, KC>(xf, ldx, 0, (int)K, lds, [&]() {
#pragma unroll
        for (int u = 0; u < DS; u++) i4_seg_load<TW>(wq[u], rows, 0, u, nsteps);
    }, prep);
    const bool bn = n < 3 * M;
    const uint8_t *bp = lds + (bn ? n : 0) * RB + 32 * kg;
    ut_i32x4 acc[TW];
#pragma unroll
    for (int w = 0; w < TW; w++) acc[w] = ut_i32x4{0, 0, 0, 0};
    auto segment = [&](uint4 (&d)[TW][2], int sg) {
        i4_seg_store<TW>(d, warea);
        i4_seg_load<TW>(d, rows, 0, sg + DS, nsteps);
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const int j = 2 * sg + s;
            if (j >= nsteps) break;
            uint4 b0 = *(const uint4 *)(bp + kMfmaStepCols * j);
            uint4 b1 = *(const uint4 *)(bp + kMfmaStepCols * j + 16);
            if (!bn) b0 = b1 = make_uint4(0u, 0u, 0u, 0u);
            const ut_i32x4 B0 = {(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w};
            const ut_i32x4 B1 = {(int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
            i4_seg_mfma<TW>(warea, s, B0, B1, acc);
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    int t = 0;
    for (; t + DS <= nseg; t += DS) {
#pragma unroll
        for (int u = 0; u < DS; u++) segment(wq[u], t + u);
    }
    for (; t < nseg; t++) {
        const int u = t % DS;
#pragma unroll
        for (int v = 0; v < DS; v++)
            if (v == u) segment(wq[v], t);
    }
#pragma unroll
    for (int w = 0; w < TW; w++) mfma_collect<M>(acc[w], res[w]);
}

// The same GEMV over a long K staged in chunks of KC columns (K % 512 ==
// 0; every chunk but the last a multiple of 4 steps): f32 activations with
// given shifts sh[m] (INT32_MIN: zero digits).  The next chunk's
// activations load into registers while the current one computes, and the
// weight loads run on across chunk boundaries (the barriers between
// chunks wait for LDS only).
// TW tiles of 16 rows per wave share each staged chunk.
template <int M, int KC, int TW>
__device__ __forceinline__ void mfma_gemv_i4_chunks(const uint8_t *const (&rows)[TW][2], int64_t K,
                                                    const float *xf, int64_t ldx,
                                                    const int32_t (&sh)[M], uint8_t *lds,
                                                    uint8_t *warea,
                                                    CoreOut<UT_FMT_INT4, M, 4> (&res)[TW]) {
    static_assert(M >= 1 && M <= 4, "three digit planes per row, 16 columns");
    static_assert(KC % (4 * kMfmaStepCols) == 0, "chunks of whole step groups");
    // segments (two steps) of weights in flight: one at two rows, two beyond
    constexpr int DS = M == 2 ? 1 : 2;
    constexpr int RB = mfma_row_bytes<KC>();
    constexpr int NI = (M * (KC / 8) + kGemvThreads - 1) / kGemvThreads;
    const int tid = threadIdx.x, lane = tid & 63, n = lane & 15, kg = lane >> 4;
    const int nsteps = (int)(K / kMfmaStepCols);
    float4 xv[NI][2];
    auto xload = [&](int64_t kc) {
        const int kcn = (int)(K - kc < KC ? K - kc : KC), NG = kcn / 8, TOT = M * NG;
#pragma unroll
        for (int j = 0; j < NI; j++) {
            const int i = tid + j * kGemvThreads, ic = i < TOT ? i : TOT - 1;
            const int m = ic / NG, g = ic - m * NG;
            const float *src = xf + m * ldx + kc + 8 * g;
            xv[j][0] = ld_global<float4>(src);
            xv[j][1] = ld_global<float4>(src + 4);
        }
    };
    auto xstore = [&](int64_t kc) {
        const int kcn = (int)(K - kc < KC ? K - kc : KC), NG = kcn / 8, TOT = M * NG;
#pragma unroll
        for (int j = 0; j < NI; j++) {
            const int i = tid + j * kGemvThreads;
            if (i < TOT) {
                const int m = i / NG, g = i - m * NG;
                const int32_t s = m == 0 ? sh[0] : m == 1 ? sh[M > 1 ? 1 : 0]
                                : m == 2 ? sh[M > 2 ? 2 : 0] : sh[M > 3 ? 3 : 0];
                const float ev[4] = {xv[j][0].x, xv[j][0].z, xv[j][1].x, xv[j][1].z};
                const float od[4] = {xv[j][0].y, xv[j][0].w, xv[j][1].y, xv[j][1].w};
                uint32_t we[3], wo[3];
                digit_words<UT_FMT_INT8>(ev, 4, s, we);
                digit_words<UT_FMT_INT8>(od, 4, s, wo);
#pragma unroll
                for (int p = 0; p < 3; p++)
                    *(uint2 *)(lds + (3 * m + p) * RB + 8 * g) = make_uint2(we[p], wo[p]);
            }
        }
    };
    auto lds_barrier = []() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };
    xload(0);
    uint4 wq[DS][TW][2];
#pragma unroll
    for (int u = 0; u < DS; u++) i4_seg_load<TW>(wq[u], rows, 0, u, nsteps);
    xstore(0);
    lds_barrier();
    const bool bn = n < 3 * M;
    const uint8_t *bp = lds + (bn ? n : 0) * RB + 32 * kg;
    ut_i32x4 acc[TW];
#pragma unroll
    for (int w = 0; w < TW; w++) acc[w] = ut_i32x4{0, 0, 0, 0};
    auto segment = [&](uint4 (&d)[TW][2], int sg, int jl) {
        i4_seg_store<TW>(d, warea);
        i4_seg_load<TW>(d, rows, 0, sg + DS, nsteps);
#pragma unroll
        for (int s = 0; s < 2; s++) {
            uint4 b0 = *(const uint4 *)(bp + kMfmaStepCols * (jl + s));
            uint4 b1 = *(const uint4 *)(bp + kMfmaStepCols * (jl + s) + 16);
            if (!bn) b0 = b1 = make_uint4(0u, 0u, 0u, 0u);
            const ut_i32x4 B0 = {(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w};
            const ut_i32x4 B1 = {(int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
            i4_seg_mfma<TW>(warea, s, B0, B1, acc);
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    int g0 = 0;  // global segment of the chunk's first
    for (int64_t kc = 0; kc < K; kc += KC) {
        const bool more = kc + KC < K;
        if (more) xload(kc + KC);
        // every chunk holds a multiple of 4 steps: whole segments, DS of them
        // per round (DS <= 2), so segment g sits in slot g % DS
        const int csegs = (int)((K - kc < KC ? K - kc : KC) / (2 * kMfmaStepCols));
        for (int t = 0; t < csegs; t += DS) {
#pragma unroll
            for (int u = 0; u < DS; u++) segment(wq[u], g0 + t + u, 2 * (t + u));
        }
        g0 += csegs;
        if (more) {
            lds_barrier();  // every wave is done with this chunk
            xstore(kc + KC);
            lds_barrier();
        }
    }
#pragma unroll
    for (int w = 0; w < TW; w++) mfma_collect<M>(acc[w], res[w]);
}

// ---------------------------------------------------------------- int8 ---
// int8 weights on the matrix cores (the dense GEMVs of 3-4-row verify steps
// and prefill chunks: the dot-product core issues 12 dot instructions per 4
// weight bytes there and is VALU-bound).  One v_mfma_i32_16x16x64_i8 per
// 64-column step and 16-row tile: A is the weights' own bytes, B the
// activations' three balanced base-256 digit planes per row (plane row
// n = 3m + p, natural column order), so the totals equal the dot-product
// core's bit for bit.
//
// Weight loads: the A operand gives a lane 16 bytes of one row (lane
// (i, kg): row i, columns [64s + 16kg, +16) of step s), so loading it
// directly asks for 64 bytes of each row per instruction, half a 128-byte
// line, and every line twice.  Instead a wave loads a 256-column segment
// of its 16 rows (four steps) as four instructions of 4 rows x 256
// contiguous bytes (lane l: row 4r + l/16, bytes 16 (l % 16)), writes them
// to a wave-private LDS area and reads the A operands back from it: with
// the loads whole lines, lm_head-sized GEMVs at four rows went from 192 to
// about 150 us in a timing-only probe of the access pattern.  The area's
// 16-byte chunks are XOR-swizzled by the row (chunk c of row i at
// 16 (c ^ i)), so the 16 rows a read touches sit in distinct banks.
//
// Columns [kb, ke) (multiples of 256) in staged chunks of KC for B; the
// next chunk's activations load into registers while the current one
// computes, and the weight loads run on across the chunk barriers.
// Activations come as digit planes (dig: [M][3][KW] words, the row
// digitiser's form) or, with F32X, as f32 rows digitised while staged with
// the shifts prep() fills (INT32_MIN: zero digits).  rows[w][r]: this
// lane's load row of tile w, instruction r (row 4r + lane/16 of the tile,
// clamped to a valid row).  DS: 256-column segments in flight.
template <int M, int KC> __host__ __device__ constexpr int mfma_i8_lds_bytes() {
    return 3 * M * mfma_row_bytes<KC>();
}
constexpr int kMfmaI8StepCols = 64;
constexpr int kMfmaI8SegCols = 256;                // four steps
constexpr int kMfmaI8WaveAreaBytes = 16 * 256;     // one segment of a 16-row tile

template <int M, int KC, int TW, int DS, bool F32X, typename Prep>
__device__ __forceinline__ void mfma_gemv_i8(const uint8_t *const (&rows)[TW][4], int64_t kb,
                                             int64_t ke, const uint32_t *dig, int64_t KW,
                                             const float *xf, int64_t ldx, uint8_t *lds,
                                             uint8_t *warea /* TW * kMfmaI8WaveAreaBytes */,
                                             CoreOut<UT_FMT_INT4, M, 4> (&res)[TW], Prep &&prep) {
    static_assert(M >= 1 && M <= 4, "three digit planes per row, 16 columns");
    static_assert(KC % kMfmaI8SegCols == 0, "chunks of whole segments");
    // a segment's slot in flight is its index mod DS across chunks
    static_assert((KC / kMfmaI8SegCols) % DS == 0, "DS divides a chunk's segments");
    constexpr int RB = mfma_row_bytes<KC>();
    // staging work items per chunk: 16-byte pieces of the 3M plane rows, or
    // 4-column groups of the M f32 rows
    constexpr int ITEMS = F32X ? M * (KC / 4) : 3 * M * (KC / 16);
    constexpr int NI = (ITEMS + kGemvThreads - 1) / kGemvThreads;
    const int tid = threadIdx.x, lane = tid & 63, n = lane & 15, kg = lane >> 4;
    const int nseg = (int)((ke - kb) / kMfmaI8SegCols);
    const int64_t lo = kb + 16 * n;  // this lane's bytes within each loaded segment
    uint4 xr[NI];
    int32_t shl[4] = {0, 0, 0, 0};
    auto xload = [&](int64_t kc) {
        const int kcn = (int)(ke - kb - kc < KC ? ke - kb - kc : KC);
        if constexpr (F32X) {
            const int NG = kcn / 4, TOT = M * NG;
#pragma unroll
            for (int j = 0; j < NI; j++) {
                const int i = tid + j * kGemvThreads, ic = i < TOT ? i : TOT - 1;
                const int m = ic / NG, g = ic - m * NG;
                const float4 v = ld_global<float4>(xf + m * ldx + kb + kc + 4 * g);
                xr[j] = make_uint4(__float_as_uint(v.x), __float_as_uint(v.y),
                                   __float_as_uint(v.z), __float_as_uint(v.w));
            }
        } else {
            const int NQ = kcn / 16, TOT = 3 * M * NQ;
#pragma unroll
            for (int j = 0; j < NI; j++) {
                const int i = tid + j * kGemvThreads, ic = i < TOT ? i : TOT - 1;
                const int r = ic / NQ, q = ic - r * NQ;
                xr[j] = ld_global<uint4>((const uint8_t *)(dig + r * KW) + kb + kc + 16 * q);
            }
        }
    };
    auto xstore = [&](int64_t kc) {
        const int kcn = (int)(ke - kb - kc < KC ? ke - kb - kc : KC);
        if constexpr (F32X) {
            const int NG = kcn / 4, TOT = M * NG;
#pragma unroll
            for (int j = 0; j < NI; j++) {
                const int i = tid + j * kGemvThreads;
                if (i < TOT) {
                    const int m = i / NG, g = i - m * NG;
                    const int32_t sh = m == 0 ? shl[0] : m == 1 ? shl[1] : m == 2 ? shl[2] : shl[3];
                    const float v[4] = {__uint_as_float(xr[j].x), __uint_as_float(xr[j].y),
                                        __uint_as_float(xr[j].z), __uint_as_float(xr[j].w)};
                    uint32_t wd[3];
                    digit_words<UT_FMT_INT8>(v, 4, sh, wd);
#pragma unroll
                    for (int p = 0; p < 3; p++) *(uint32_t *)(lds + (3 * m + p) * RB + 4 * g) = wd[p];
                }
            }
        } else {
            const int NQ = kcn / 16, TOT = 3 * M * NQ;
#pragma unroll
            for (int j = 0; j < NI; j++) {
                const int i = tid + j * kGemvThreads;
                if (i < TOT) {
                    const int r = i / NQ, q = i - r * NQ;
                    *(uint4 *)(lds + r * RB + 16 * q) = xr[j];
                }
            }
        }
    };
    auto lds_barrier = []() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };
    // the segment in flight: wq[slot][w][r] = tile w's rows 4r + lane/16
    uint4 wq[DS][TW][4];
    auto seg_load = [&](uint4 (&d)[TW][4], int sg) {
        const int64_t off = lo + (int64_t)kMfmaI8SegCols * (sg < nseg ? sg : nseg - 1);
#pragma unroll
        for (int w = 0; w < TW; w++)
#pragma unroll
            for (int r = 0; r < 4; r++) d[w][r] = ld_weights(rows[w][r] + off);
    };
    xload(0);
#pragma unroll
    for (int u = 0; u < DS; u++) seg_load(wq[u], u);
    __builtin_amdgcn_sched_barrier(0);
    prep(shl);
    xstore(0);
    lds_barrier();
    const bool bn = n < 3 * M;
    const uint8_t *bp = lds + (bn ? n : 0) * RB + 16 * kg;
    // A reads: row n, chunk 4s + kg at 16 ((4s + kg) ^ n); writes: row
    // 4r + kg, chunk n at 16 (n ^ (4r + kg))
    ut_i32x4 acc[TW];
#pragma unroll
    for (int w = 0; w < TW; w++) acc[w] = ut_i32x4{0, 0, 0, 0};
    auto segment = [&](uint4 (&d)[TW][4], int sg, int sl) {
#pragma unroll
        for (int w = 0; w < TW; w++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = 4 * r + kg;
                *(uint4 *)(warea + w * kMfmaI8WaveAreaBytes + row * 256 + 16 * (n ^ row)) = d[w][r];
            }
        seg_load(d, sg + DS);
#pragma unroll
        for (int s = 0; s < 4; s++) {
            uint4 b = *(const uint4 *)(bp + kMfmaI8SegCols * sl + kMfmaI8StepCols * s);
            if (!bn) b = make_uint4(0u, 0u, 0u, 0u);
            const ut_i32x4 B = {(int)b.x, (int)b.y, (int)b.z, (int)b.w};
#pragma unroll
            for (int w = 0; w < TW; w++) {
                const uint4 av = *(const uint4 *)(warea + w * kMfmaI8WaveAreaBytes + n * 256 +
                                                  16 * ((4 * s + kg) ^ n));
                const ut_i32x4 A = {(int)av.x, (int)av.y, (int)av.z, (int)av.w};
                acc[w] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, acc[w], 0, 0, 0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    int g0 = 0;  // the chunk's first segment
    for (int64_t kc = 0; kc < ke - kb; kc += KC) {
        const bool more = kc + KC < ke - kb;
        if (more) xload(kc + KC);
        const int csegs = (int)((ke - kb - kc < KC ? ke - kb - kc : KC) / kMfmaI8SegCols);
        int t = 0;
        // every chunk but the last holds KC / 256 segments, a multiple of DS,
        // so segment g sits in slot g % DS
        for (; t + DS <= csegs; t += DS) {
#pragma unroll
            for (int u = 0; u < DS; u++) segment(wq[u], g0 + t + u, t + u);
        }
        for (; t < csegs; t++) {
            const int u = (g0 + t) % DS;
#pragma unroll
            for (int v = 0; v < DS; v++)
                if (v == u) segment(wq[v], g0 + t, t);
        }
        g0 += csegs;
        if (more) {
            lds_barrier();  // every wave is done with this chunk
            xstore(kc + KC);
            lds_barrier();
        }
    }
#pragma unroll
    for (int w = 0; w < TW; w++) mfma_collect<M>(acc[w], res[w]);
}

}  // namespace ut
