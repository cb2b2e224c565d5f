// ut_mla.hip -- absorbed-MLA decode attention core on gfx950
// (adapters/undertow-deepseek-moe/src/attention.rs:214-234): for R query
// rows x H heads over the shared latent cache, split-T flash decoding.
//
//   k_mla_split    grid (R*H/HG, nsplit): a workgroup takes HG heads of one
//                  query row and one 64-position slice of the cache; a lane
//                  scores one position against HG/4 queries, then the
//                  slice's max / sum / unnormalised context are written out.
//   k_mla_combine  merges the slices: M = max m_j, L = sum l_j e^(m_j-M),
//                  clat = sum o_j e^(m_j-M) / L.
// Row s sees n_ctx = pos_base + s + 1 positions.  Slice boundaries depend
// only on the position index, so a row's result does not depend on R.
// Scores accumulate as the reference does: sum_i q_i*lat_i then
// sum_i qr_i*krot_i, sequential f32 adds without contraction.
#include "ut_internal.h"
#include "ut_mla.h"

namespace ut {

constexpr int kMlaSlice = 64;

// Workgroup = HG heads of one query row x one 64-position slice.
// Scores: wave w takes heads w, w+4, ... (HG/4 of them), lane = position;
// the slice max / sum per head are wave reductions.  Context: thread t takes
// latent columns t, t+256, ... for all HG heads over the slice.
template <int HG>
__global__ __launch_bounds__(256) void k_mla_split(const float *__restrict__ qabs,
                                                   const float *__restrict__ qrope,
                                                   const float *__restrict__ latent,
                                                   const float *__restrict__ krot, int R, int H,
                                                   int L, int P, PosRef pos, float scale,
                                                   float *__restrict__ part_m,
                                                   float *__restrict__ part_l,
                                                   float *__restrict__ part_o, int nsplit) {
    extern __shared__ float sm[];
    constexpr int HW = HG >= 4 ? HG / 4 : 1;  // heads per wave
    const int QW = L + P;
    float *q = sm;                  // [HG][L + P]
    float *p = sm + HG * QW;        // [HG][kMlaSlice]
    const int groups = H / HG;
    const int r = blockIdx.x / groups, h0 = (blockIdx.x % groups) * HG;
    const int j = blockIdx.y, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int64_t n_ctx = pos.get() + r + 1;
    const int64_t t0 = (int64_t)j * kMlaSlice;
    // past the row's context (a grid sized for more positions): the combine
    // reads only the row's own slices
    if (t0 >= n_ctx) return;
    for (int i = tid; i < HG * QW; i += 256) {
        int hh = i / QW, d = i - hh * QW;
        int64_t qi = ((int64_t)r * H + h0 + hh);
        q[i] = d < L ? qabs[qi * L + d] : qrope[qi * P + (d - L)];
    }
    __syncthreads();
    const int64_t pb = ((int64_t)r * H + h0) * nsplit + j;  // part index of head h0
    if (wave < HG) {
        const int64_t pos = t0 + lane;
        const bool live = pos < n_ctx;
        float sc[HW];
#pragma unroll
        for (int k = 0; k < HW; k++) sc[k] = 0.0f;
        if (live) {
            // score = sum_i q_i*lat_i + sum_i qr_i*krot_i, sequential adds
            const float *lr = latent + pos * L;
#pragma unroll 8
            for (int d = 0; d < L; d += 4) {
                const float4 kv = *(const float4 *)(lr + d);
#pragma unroll
                for (int k = 0; k < HW; k++) {
                    const float *qq = q + (wave + 4 * k) * QW + d;
                    float a = sc[k];
                    a = __fadd_rn(a, __fmul_rn(qq[0], kv.x));
                    a = __fadd_rn(a, __fmul_rn(qq[1], kv.y));
                    a = __fadd_rn(a, __fmul_rn(qq[2], kv.z));
                    a = __fadd_rn(a, __fmul_rn(qq[3], kv.w));
                    sc[k] = a;
                }
            }
            const float *kr = krot + pos * P;
#pragma unroll 8
            for (int d = 0; d < P; d++) {
                const float kv = kr[d];
#pragma unroll
                for (int k = 0; k < HW; k++)
                    sc[k] = __fadd_rn(sc[k], __fmul_rn(q[(wave + 4 * k) * QW + L + d], kv));
            }
        }
#pragma unroll
        for (int k = 0; k < HW; k++) {
            const int hh = wave + 4 * k;
            if (hh >= HG) break;
            const float v = live ? __fmul_rn(sc[k], scale) : -INFINITY;
            float mx = v;
            for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
            const float e = live ? expf(v - mx) : 0.0f;
            p[hh * kMlaSlice + lane] = e;
            float sum = e;
            for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, 64);
            if (lane == 0) {
                part_m[pb + (int64_t)hh * nsplit] = mx;
                part_l[pb + (int64_t)hh * nsplit] = sum;
            }
        }
    }
    __syncthreads();
    // unnormalised context over the slice
    const int64_t tn = n_ctx - t0 < kMlaSlice ? n_ctx - t0 : kMlaSlice;
    for (int d = tid; d < L; d += 256) {
        float o[HG];
#pragma unroll
        for (int hh = 0; hh < HG; hh++) o[hh] = 0.0f;
#pragma unroll 16
        for (int64_t t = 0; t < tn; t++) {
            const float kv = latent[(t0 + t) * L + d];
#pragma unroll
            for (int hh = 0; hh < HG; hh++) o[hh] = __builtin_fmaf(p[hh * kMlaSlice + t], kv, o[hh]);
        }
#pragma unroll
        for (int hh = 0; hh < HG; hh++) part_o[(pb + (int64_t)hh * nsplit) * L + d] = o[hh];
    }
}

__global__ __launch_bounds__(256) void k_mla_combine(const float *__restrict__ part_m,
                                                     const float *__restrict__ part_l,
                                                     const float *__restrict__ part_o, int L,
                                                     int H, PosRef pos, int nsplit,
                                                     float *__restrict__ clat) {
    const int64_t qi = blockIdx.x;  // r*H + h
    const int r = (int)(qi / H);
    const int64_t n_ctx = pos.get() + r + 1;
    const int ns = (int)((n_ctx + kMlaSlice - 1) / kMlaSlice);
    float M = -INFINITY;
#pragma unroll 8
    for (int j = 0; j < ns; j++) M = fmaxf(M, part_m[qi * nsplit + j]);
    float Lsum = 0.0f;
    for (int j = 0; j < ns; j++) Lsum = __fadd_rn(Lsum, __fmul_rn(part_l[qi * nsplit + j], expf(part_m[qi * nsplit + j] - M)));
    const float inv = 1.0f / Lsum;
    for (int d = threadIdx.x; d < L; d += 256) {
        float acc = 0.0f;
#pragma unroll 8
        for (int j = 0; j < ns; j++)
            acc = __builtin_fmaf(part_o[(qi * nsplit + j) * L + d], expf(part_m[qi * nsplit + j] - M), acc);
        clat[qi * L + d] = __fmul_rn(acc, inv);
    }
}

// ------------------------------------------------------ MFMA variant ---
// For the DeepSeek-V3 shape (heads % 32 == 0, latent 512 + rope 64) the
// score and context contractions run on the bf16 matrix cores.  Each f32
// operand x is split into x_hi = bf16(x) and x_lo = bf16(x - x_hi), and a
// product is taken as hi*hi + hi*lo + lo*hi (f32 accumulation), which keeps
// about 16 significant bits per product term instead of bf16's 8.  The
// cache is kept in that split form ([T][2][L+P] bf16: the hi plane, then
// the lo plane of each position).
//
// Work split.  A column is one (query row r, head h) pair, c = r*H + h; a
// workgroup (k_mla_mfma16) takes 32 columns of one query row and one slice
// of positions, 16 positions per tile:
//   copy    the tile's 16 cache rows (36 KiB) go straight from global
//           memory to LDS (global_load_lds), double-buffered: the next
//           tile's copy is issued between this tile's score steps;
//   scores  S^T[pos x col] = K[pos x (L+P)] . Q^T[(L+P) x col] with
//           v_mfma_f32_16x16x32_bf16; wave w takes column block w&1 over
//           dim half w>>1 (queries held in registers), the two halves are
//           summed through LDS;
//   softmax online, per column; the exponent offset moves only when a
//           score exceeds it by more than kMlaHeadroom (so the context is
//           rescaled on such jumps only);
//   context O^T[L x col] += V^T[L x pos] . P[pos x col] with
//           v_mfma_f32_32x32x16_bf16; wave w owns latent dims
//           [128w, 128w + 128); V^T comes from the tile's rows in LDS by the
//           transposing read (ds_read_b64_tr_b16: within each 16-lane group,
//           lane j supplies 4 consecutive dims of row 4q + j/4 and lane i
//           receives dim i of the group's 4 rows).
// LDS has 64 banks (256 bytes per pass: 16 lanes of a 16-byte read, 32
// lanes of an 8-byte read).  Every 2,304-byte row starts at bank 0, so a
// row's 16-byte chunks are XOR-swizzled by mla_swz(r), a 4-bit permutation
// of the row index (chunk groups of 16 stay inside the 144-chunk row):
// the score read's 16 lanes (rows 0-15, one chunk) get 16 distinct slots,
// and the transposing read's 32 lanes (4 consecutive rows x 4 chunks of a
// 4-aligned group) too, since rows 4k..4k+3 differ in the swizzle's high
// two bits.  The score exchange rows are padded to 20 floats (80-byte
// stride: 16 lanes at distinct 16-byte slots).
// 77 KiB of LDS and < 256 registers per lane let two workgroups share a CU.
// The slice writes (m, l, O) to the partial buffers, k_mla_combine_mfma
// merges the slices.  The slice length depends only on the row's context
// length, so a row's result is the same whichever rows share the call.
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));


// Slice length of a row that sees n_ctx positions: about n_ctx/64 in whole
// 16-position tiles, at least 32 and at most UT_MLA_SLICE_CAP = 512 (so at
// most 64 slices up to 32768 positions, n_ctx/512 beyond).  A function of
// n_ctx alone, so a row's result does not depend on which rows share the
// call; no power-of-two steps, so neighbouring context lengths get similar
// slice counts.  The cap of 512 against 256 halves the slice partials past
// 16384 positions: at T = 32768 two- and four-row calls went from 97.2 to
// 88.0 us and from 179.3 to 154.6 us, one-row calls from 56.6 to 61.1 us
// (256 workgroups, one per CU).  Verify rows outnumber single rows in
// speculative decoding (every main-model layer of a round), so 512.
#ifndef UT_MLA_SLICE_CAP
#define UT_MLA_SLICE_CAP 512
#endif
__host__ __device__ inline int64_t mla_mfma_slice(int64_t n_ctx) {
    const int64_t s = (n_ctx + 1023) / 1024 * 16;
    return s < 32 ? 32 : s > UT_MLA_SLICE_CAP ? UT_MLA_SLICE_CAP : s;
}

__device__ __forceinline__ void split8(const float (&x)[8], bf16x8_t &hi, bf16x8_t &lo) {
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const __bf16 h = (__bf16)x[j];
        hi[j] = h;
        lo[j] = (__bf16)__fsub_rn(x[j], (float)h);
    }
}

__device__ __forceinline__ void load8(const float *p, float (&x)[8]) {
    const float4 a = *(const float4 *)p, b = *(const float4 *)(p + 4);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}

struct MlaMfmaArgs {
    const float *qabs, *qrope;
    const __bf16 *kc;  // [T][2][L+P]: bf16 hi plane then lo plane per position
    int H, L, P, RH;
    PosRef pos;
    float scale;
    int groups, nslice;  // column groups of 32, slices in the grid
    float *part_m, *part_l, *part_o;  // [j][col], [j][col], [j][L][col]
};

constexpr int kRowChunks = 144;       // 16-byte chunks per position (576 hi + 576 lo)
constexpr float kMlaHeadroom = 8.0f;  // nats a score may exceed the running offset

__device__ __forceinline__ int mla_swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }
__device__ __forceinline__ int mla_slot(int r, int c) { return r * kRowChunks + (c ^ mla_swz(r)); }

typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf16x4_t lds_bf16x4_t;
__device__ __forceinline__ bf16x8_t tr_pair(const uint8_t *lds_a, const uint8_t *lds_b) {
    const bf16x4_t x = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
        (lds_bf16x4_t *)(__attribute__((address_space(3))) uint8_t *)lds_a);
    const bf16x4_t y = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
        (lds_bf16x4_t *)(__attribute__((address_space(3))) uint8_t *)lds_b);
    return __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Lanes l and l ^ 32 combined without an LDS round trip: permlane32_swap
// of (v, v) returns the low halves of both operands in one register and the
// high halves in the other, so max / sum of the two is the pair's result in
// every lane (and the same sum order in both lanes).
__device__ __forceinline__ float pair_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __fadd_rn(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

constexpr int kTile16 = 16;
constexpr int kTile16Bytes = kTile16 * kRowChunks * 16;  // 36864

__global__ __launch_bounds__(256, 2) void k_mla_mfma16(MlaMfmaArgs a) {
    constexpr int KS = 9, MT = 4, D = 576;
    typedef __bf16 bf16x8l_t __attribute__((ext_vector_type(8)));
    typedef float f32x4l_t __attribute__((ext_vector_type(4)));
    __shared__ __attribute__((aligned(16))) uint8_t sT0[kTile16Bytes];
    __shared__ __attribute__((aligned(16))) uint8_t sT1[kTile16Bytes];
    // [dim half][column][position], rows padded to 20 floats
    __shared__ __attribute__((aligned(16))) float sS[2][32][kTile16 + 4];
    const int b = blockIdx.x, x8 = b & 7, q = b >> 3;
    const int group = q % a.groups;
    const int slice = (q / a.groups) * 8 + x8;
    const int c0 = group * 32;
    const int r = c0 / a.H;
    const int64_t n_ctx = a.pos.get() + r + 1;
    const int64_t slen = mla_mfma_slice(n_ctx);
    const int64_t p0 = (int64_t)slice * slen;
    if (slice >= a.nslice || p0 >= n_ctx) return;  // uniform per workgroup
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
    const int cb = w & 1, dh = w >> 1;
    const int L = a.L, P = a.P;
    // score operand lanes: column 16*cb + (l & 15), dims 288*dh + 32*ks + 8*(l >> 4)
    const int qcol = c0 + 16 * cb + (l & 15);
    const int qd0 = 288 * dh + 8 * (l >> 4);
    bf16x8l_t qh[KS], ql[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
        const int d0 = qd0 + 32 * ks;
        float v[8];
        load8(d0 < L ? a.qabs + (int64_t)qcol * L + d0 : a.qrope + (int64_t)qcol * P + (d0 - L), v);
        split8(v, qh[ks], ql[ks]);
    }
    // context lanes: column l & 31, positions 8*(l >> 5) + [0, 8)
    const int n = l & 31, kh = l >> 5;
    const int col = c0 + n;
    f32x16_t o[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int i = 0; i < 16; i++) o[mt][i] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;
    const int64_t tend = p0 + slen < n_ctx ? p0 + slen : n_ctx;
    const uint32_t last = (uint32_t)(n_ctx - 1);

    // wave w copies slots [w*9*64, (w+1)*9*64) of a tile (part i: one 1 KiB run)
    auto copy_part = [&](uint32_t t0, uint8_t *dst, int i) {
        const int s0 = (w * 9 + i) * 64, sl = s0 + l;
        const int rr = sl / kRowChunks, phy = sl - rr * kRowChunks;
        const int c = phy ^ mla_swz(rr);
        const uint32_t pos = t0 + rr <= last ? t0 + rr : last;
        const __bf16 *src = a.kc + (size_t)pos * (2 * D) + c * 8;
        __builtin_amdgcn_global_load_lds((const void *)src,
                                         (__attribute__((address_space(3))) void *)(dst + s0 * 16),
                                         16, 0, 0);
    };
#pragma unroll
    for (int i = 0; i < 9; i++) copy_part((uint32_t)p0, sT0, i);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();

    auto tile = [&](const uint8_t *T, uint8_t *Nx, int64_t t0) {
        const bool more = t0 + kTile16 < tend;
        const uint32_t tn = (uint32_t)(t0 + kTile16);
        // ---- partial scores: 16 positions x this wave's 16 columns, its dim half
        // three independent accumulator chains (hi*hi, hi*lo, lo*hi), summed
        // at the end, keep the matrix pipe busy
        f32x4l_t sa = {0.0f, 0.0f, 0.0f, 0.0f}, sb = sa, sd = sa;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            if (more) copy_part(tn, Nx, ks);
            const int ch = 36 * dh + 4 * ks + (l >> 4);
            const bf16x8l_t kh8 = *(const bf16x8l_t *)(T + mla_slot(l & 15, ch) * 16);
            const bf16x8l_t kl8 = *(const bf16x8l_t *)(T + mla_slot(l & 15, 72 + ch) * 16);
            sa = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh8, qh[ks], sa, 0, 0, 0);
            sb = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh8, ql[ks], sb, 0, 0, 0);
            sd = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kl8, qh[ks], sd, 0, 0, 0);
        }
        f32x4l_t sc;
#pragma unroll
        for (int i = 0; i < 4; i++) sc[i] = __fadd_rn(sa[i], __fadd_rn(sb[i], sd[i]));
        // C layout: register i holds position 4*(l >> 4) + i, column l & 15
        *(f32x4l_t *)&sS[dh][16 * cb + (l & 15)][4 * (l >> 4)] = sc;
        // an LDS-only barrier (the fence of __syncthreads would also wait
        // for the next tile's copy)
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        // ---- this lane's 8 positions of column n, dim halves summed in order
        const f32x4l_t a0 = *(const f32x4l_t *)&sS[0][n][8 * kh];
        const f32x4l_t a1 = *(const f32x4l_t *)&sS[0][n][8 * kh + 4];
        const f32x4l_t b0 = *(const f32x4l_t *)&sS[1][n][8 * kh];
        const f32x4l_t b1 = *(const f32x4l_t *)&sS[1][n][8 * kh + 4];
        const int live = n_ctx - t0 < kTile16 ? (int)(n_ctx - t0) : kTile16;
        float p[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float v = __fadd_rn(e < 4 ? a0[e] : a1[e - 4], e < 4 ? b0[e] : b1[e - 4]);
            p[e] = __fadd_rn(__fmul_rn(v, a.scale), 8 * kh + e < live ? 0.0f : -INFINITY);
        }
        float mt_ = p[0];
#pragma unroll
        for (int e = 1; e < 8; e++) mt_ = fmaxf(mt_, p[e]);
        mt_ = pair_max(mt_);
        // the exponent offset moves only on a jump of more than kMlaHeadroom
        const bool jump = mt_ > m_run + kMlaHeadroom;
        const float m_new = jump ? mt_ : m_run;
        if (__any(jump)) {
            const float alpha = __expf(m_run - m_new);
            l_run *= alpha;
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int i = 0; i < 16; i++) o[mt][i] *= alpha;
        }
        float ls = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            p[e] = __expf(p[e] - m_new);
            ls += p[e];
        }
        ls = pair_sum(ls);
        l_run += ls;
        m_run = m_new;
        bf16x8_t ph, pl;
        split8(p, ph, pl);
        // ---- context over this wave's 128 latent dims (k = the 16 positions)
        const int g = l >> 4, j = l & 15;
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const int d0 = 128 * w + 32 * mt + 16 * (g & 1);
            const int chunk = (d0 >> 3) + ((j & 3) >> 1), boff = 8 * (j & 1);
            const int ra = 8 * kh + (j >> 2), rb = ra + 4;
            const bf16x8_t vh = tr_pair(T + mla_slot(ra, chunk) * 16 + boff,
                                        T + mla_slot(rb, chunk) * 16 + boff);
            const bf16x8_t vl = tr_pair(T + mla_slot(ra, 72 + chunk) * 16 + boff,
                                        T + mla_slot(rb, 72 + chunk) * 16 + boff);
            o[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vh, ph, o[mt], 0, 0, 0);
            o[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vh, pl, o[mt], 0, 0, 0);
            o[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vl, ph, o[mt], 0, 0, 0);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    };
    for (int64_t t0 = p0; t0 < tend; t0 += 2 * kTile16) {
        tile(sT0, sT1, t0);
        if (t0 + kTile16 < tend) tile(sT1, sT0, t0 + kTile16);
    }
    // ---- slice partials: O^T register i is dim 128*w + 32*mt + (i/4)*8 + kh*4 + i%4
    const int64_t RH = a.RH;
    if (w == 0 && kh == 0) {
        a.part_m[(int64_t)slice * RH + col] = m_run;
        a.part_l[(int64_t)slice * RH + col] = l_run;
    }
    float *po = a.part_o + ((int64_t)slice * L + 128 * w + kh * 4) * RH + col;
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int i = 0; i < 16; i++)
            po[(int64_t)(32 * mt + (i >> 2) * 8 + (i & 3)) * RH] = o[mt][i];
}

// The cache in the MFMA kernel's form: per position the bf16 hi parts of
// [latent | k_rot] then the lo parts, x = hi + lo + O(2^-17 |x|).
__global__ __launch_bounds__(256) void k_mla_cache_split(const float *__restrict__ latent,
                                                         const float *__restrict__ krot, int L,
                                                         int P, int64_t T,
                                                         __bf16 *__restrict__ kc) {
    const int D = L + P;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= T * D) return;
    const int64_t pos = i / D;
    const int d = (int)(i - pos * D);
    const float x = d < L ? latent[pos * L + d] : krot[pos * P + (d - L)];
    const __bf16 h = (__bf16)x;
    kc[pos * 2 * D + d] = h;
    kc[pos * 2 * D + D + d] = (__bf16)__fsub_rn(x, (float)h);
}

// Merges the slices: M = max m_j, Ls = sum l_j e^(m_j - M),
// clat = sum_j o_j e^(m_j - M) / Ls.  A workgroup takes 32 columns x 8 dims;
// thread (col, t) first takes slices j = t, t+8, ... for the max and the
// weights (kept in LDS; partial sums reduced in t order), then dim t over
// all slices.  Every sum runs in a fixed order.
constexpr int kMlaMaxSlices = 256;

// A workgroup merges 32 columns x 8 latent dims, as 1,024 virtual threads
// (NT threads, each standing for 1024 / NT of them).  Every load is issued
// at the start (one memory round trip): virtual thread (tx, tyz) holds the
// slice statistics m, l of column tx for slices tyz + 32k; virtual thread
// (c4, dy, part) holds four adjacent columns of dim dy (16-byte loads) for
// one sixteenth of the slices.  The 32 statistic sums and the sixteen part
// sums are added in index order through LDS, so every output's sum has a
// fixed order and NT does not change a bit of the result.
// MAXS: the most slices the instantiation takes (the register arrays are
// sized for it; with 64, two workgroups fit a CU instead of one).  Any
// MAXS >= the rows' slice count runs the same operations in the same order.
// NT < 1024 (fewer, busier threads) lets more rows' workgroups share a CU.
constexpr int kCombineParts = 16;
constexpr int kCombineSmallSlices = 64;
#ifndef UT_MLA_COMBINE_SMALL_NT
#define UT_MLA_COMBINE_SMALL_NT 256
#endif

template <int MAXS, int NT>
__global__ __launch_bounds__(NT) void k_mla_combine_mfma(const float *__restrict__ part_m,
                                                         const float *__restrict__ part_l,
                                                         const float *__restrict__ part_o,
                                                         int RH, int H, int L, PosRef pos,
                                                         float *__restrict__ clat) {
    static_assert(NT % 64 == 0 && 1024 % NT == 0 && NT >= 256, "whole waves, 256 outputs");
    constexpr int VT = 1024 / NT;                                               // virtual per thread
    constexpr int kCombineStat = MAXS / 32;                                     // m, l per vthread
    constexpr int kCombineSlices = (MAXS + kCombineParts - 1) / kCombineParts;  // per part
    __shared__ __attribute__((aligned(16))) float sw[MAXS][32];
    __shared__ float red[32][33];
    __shared__ float sM[32], sInv[32];
    __shared__ __attribute__((aligned(16))) float sq[kCombineParts][8][32];
    const int tid = threadIdx.x;
    // virtual thread tid + NT i: tx and (c4, dy) are tid's, tyz and part step
    const int tx = tid & 31, ty0 = tid >> 5;
    const int col = blockIdx.x * 32 + tx;
    // the slice count is the same for the workgroup's 32 columns (one query
    // row: 32 | H)
    const int64_t n_ctx = pos.get() + col / H + 1;
    const int64_t slen = mla_mfma_slice(n_ctx);
    const int ns = (int)((n_ctx + slen - 1) / slen);
    // merge-pass loads: columns 4*c4.., dim dy, slices [j0, j1) of each part
    const int c4 = tid & 7, dy = (tid >> 3) & 7, p0 = tid >> 6;
    const int q = (ns + kCombineParts - 1) / kCombineParts;
    const float *po = part_o + (int64_t)(blockIdx.y * 8 + dy) * RH + blockIdx.x * 32 + 4 * c4;
    const int64_t js = (int64_t)L * RH;
    float4 v[VT][kCombineSlices];
#pragma unroll
    for (int i = 0; i < VT; i++) {
        const int j0 = (p0 + (NT / 64) * i) * q, j1 = j0 + q < ns ? j0 + q : ns;
#pragma unroll
        for (int u = 0; u < kCombineSlices; u++)
            if (u < q) {
                const int j = j0 + u < j1 ? j0 + u : (j1 > 0 ? j1 - 1 : 0);
                v[i][u] = *(const float4 *)(po + (int64_t)j * js);
            }
    }
    // statistics loads
    float pm[VT][kCombineStat], pl[VT][kCombineStat];
#pragma unroll
    for (int i = 0; i < VT; i++)
#pragma unroll
        for (int k = 0; k < kCombineStat; k++) {
            const int j = ty0 + (NT / 32) * i + 32 * k;
            if (j < ns) {
                pm[i][k] = part_m[(int64_t)j * RH + col];
                pl[i][k] = part_l[(int64_t)j * RH + col];
            }
        }
#pragma unroll
    for (int i = 0; i < VT; i++) {
        const int tyz = ty0 + (NT / 32) * i;
        float mx = -INFINITY;
#pragma unroll
        for (int k = 0; k < kCombineStat; k++)
            if (tyz + 32 * k < ns) mx = fmaxf(mx, pm[i][k]);
        red[tyz][tx] = mx;
    }
    __syncthreads();
    if (ty0 == 0) {
        float M = red[0][tx];
        for (int t = 1; t < 32; t++) M = fmaxf(M, red[t][tx]);
        sM[tx] = M;
    }
    __syncthreads();
    const float M = sM[tx];
#pragma unroll
    for (int i = 0; i < VT; i++) {
        const int tyz = ty0 + (NT / 32) * i;
        float ls = 0.0f;
#pragma unroll
        for (int k = 0; k < kCombineStat; k++) {
            const int j = tyz + 32 * k;
            if (j < ns) {
                const float e = __expf(pm[i][k] - M);
                sw[j][tx] = e;
                ls = __fadd_rn(ls, __fmul_rn(pl[i][k], e));
            }
        }
        red[tyz][tx] = ls;
    }
    __syncthreads();  // sw and red complete
    if (ty0 == 0) {
        float t = red[0][tx];
        for (int u = 1; u < 32; u++) t = __fadd_rn(t, red[u][tx]);
        sInv[tx] = 1.0f / t;  // read after the barrier below
    }
#pragma unroll
    for (int i = 0; i < VT; i++) {
        const int part = p0 + (NT / 64) * i;
        const int j0 = part * q, j1 = j0 + q < ns ? j0 + q : ns;
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int u = 0; u < kCombineSlices; u++)
            if (j0 + u < j1) {
                const float4 w = *(const float4 *)&sw[j0 + u][4 * c4];
                acc.x = __builtin_fmaf(v[i][u].x, w.x, acc.x);
                acc.y = __builtin_fmaf(v[i][u].y, w.y, acc.y);
                acc.z = __builtin_fmaf(v[i][u].z, w.z, acc.z);
                acc.w = __builtin_fmaf(v[i][u].w, w.w, acc.w);
            }
        *(float4 *)&sq[part][dy][4 * c4] = acc;
    }
    __syncthreads();
    if (tid < 256) {
        const int oc = tid & 31, od = tid >> 5;  // output column, dim
        float t = sq[0][od][oc];
#pragma unroll
        for (int u = 1; u < kCombineParts; u++) t = __fadd_rn(t, sq[u][od][oc]);
        clat[(int64_t)(blockIdx.x * 32 + oc) * L + blockIdx.y * 8 + od] = __fmul_rn(t, sInv[oc]);
    }
}

// Largest slice count over the rows' context lengths n <= T (an upper
// bound: slices past a row's count exit at once).
static int64_t mla_mfma_nslice(int64_t T) {
    if (T <= 2048) return (T + 31) / 32;  // 32-position slices
    if (T <= 64 * UT_MLA_SLICE_CAP) return 64;  // length >= n/64
    return (T + UT_MLA_SLICE_CAP - 1) / UT_MLA_SLICE_CAP;  // slices of the cap
}

static bool mla_mfma_ok(int64_t H, int64_t L, int64_t P, int64_t T) {
    // instantiated for the DeepSeek-V3 MLA shape: latent 512 + rope 64
    return H % 32 == 0 && L == 512 && P == 64 && mla_mfma_nslice(T) <= kMlaMaxSlices;
}

bool mla_kc_ok(int64_t H, int64_t L, int64_t P, int64_t T) { return mla_mfma_ok(H, L, P, T); }

static size_t mla_mfma_scratch_bytes(int64_t R, int64_t H, int64_t L, int64_t T) {
    const size_t ns = (size_t)mla_mfma_nslice(T), RH = (size_t)(R * H);
    return ((ns * RH * 4 + 255) & ~size_t(255)) * 2 + ((ns * L * RH * 4 + 255) & ~size_t(255));
}

static size_t mla_split_scratch_bytes(int64_t R, int64_t H, int64_t L, int64_t T) {
    int64_t ns = (T + kMlaSlice - 1) / kMlaSlice;
    size_t n = (size_t)R * H * ns;
    size_t b = ((n * 4 + 255) & ~size_t(255)) * 2 + ((n * L * 4 + 255) & ~size_t(255));
    return b;
}

size_t mla_scratch_bytes(int64_t R, int64_t H, int64_t L, int64_t P, int64_t T) {
    // the f32 entry also holds the split cache (T x (L+P) x 4 bytes)
    return mla_mfma_ok(H, L, P, T)
               ? mla_mfma_scratch_bytes(R, H, L, T) + (size_t)T * (L + P) * 4 + 256
               : mla_split_scratch_bytes(R, H, L, T);
}

size_t mla_kc_scratch_bytes(int64_t R, int64_t H, int64_t L, int64_t T) {
    return mla_mfma_scratch_bytes(R, H, L, T);
}

int32_t launch_mla_cache_split(ut_ctx *ctx, const float *latent, const float *krot, int64_t T,
                               int64_t L, int64_t P, __bf16 *kc) {
    if (T <= 0) return UT_OK;
    const int64_t n = T * (L + P);
    int tok = timing_begin(ctx, "mla_cache_split");
    hipLaunchKernelGGL(k_mla_cache_split, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       ctx->stream, latent, krot, (int)L, (int)P, T, kc);
    timing_end(ctx, tok);
    return launch_check(ctx, "k_mla_cache_split");
}

int32_t launch_mla_attend_kc(ut_ctx *ctx, const float *qabs, const float *qrope, const __bf16 *kc,
                             int64_t R, int64_t H, int64_t L, int64_t P, int64_t pos_base,
                             float scale, float *clat, void *scratch) {
    const int64_t T = pos_extent(ctx, pos_base + R);
    if (!mla_mfma_ok(H, L, P, T) || ((uintptr_t)kc & 15) != 0) {
        set_error(ctx, "mla: split-cache attention needs 32k heads, latent 512 + rope 64, a "
                       "16-byte aligned cache and at most %d slices", kMlaMaxSlices);
        return UT_ERR_SHAPE;
    }
    const int64_t RH = R * H, ns = mla_mfma_nslice(T);
    MlaMfmaArgs a;
    a.qabs = qabs; a.qrope = qrope; a.kc = kc;
    a.H = (int)H; a.L = (int)L; a.P = (int)P; a.RH = (int)RH;
    a.pos = pos_ref(ctx, pos_base);
    a.scale = scale;
    a.groups = (int)(RH / 32);
    a.nslice = (int)ns;
    a.part_m = (float *)scratch;
    a.part_l = (float *)((char *)scratch + ((ns * RH * 4 + 255) & ~int64_t(255)));
    a.part_o = (float *)((char *)a.part_l + ((ns * RH * 4 + 255) & ~int64_t(255)));
    a.groups = (int)(RH / 32);  // 32 columns per workgroup
    const int64_t nwg = (int64_t)a.groups * ((ns + 7) / 8 * 8);
    int tok = timing_begin(ctx, "mla_mfma");
    hipLaunchKernelGGL(k_mla_mfma16, dim3((unsigned)nwg), dim3(256), 0, ctx->stream, a);
    timing_end(ctx, tok);
    UT_TRY(launch_check(ctx, "k_mla_mfma"));
    tok = timing_begin(ctx, "mla_combine");
    const dim3 cgrid((unsigned)(RH / 32), (unsigned)(L / 8));
    // up to 64 slices: 256-thread workgroups once the grid exceeds one per
    // CU (config-4 verify of four rows: 15.2 -> 7.4 us per combine; at one
    // row the 1,024-thread form is 0.2 us faster)
    if (a.nslice <= kCombineSmallSlices && (int64_t)cgrid.x * cgrid.y > ctx->multiprocessors)
        hipLaunchKernelGGL((k_mla_combine_mfma<kCombineSmallSlices, UT_MLA_COMBINE_SMALL_NT>), cgrid,
                           dim3(UT_MLA_COMBINE_SMALL_NT), 0, ctx->stream, a.part_m, a.part_l,
                           a.part_o, (int)RH, (int)H, (int)L, a.pos, clat);
    else if (a.nslice <= kCombineSmallSlices)
        hipLaunchKernelGGL((k_mla_combine_mfma<kCombineSmallSlices, 1024>), cgrid, dim3(1024), 0,
                           ctx->stream, a.part_m, a.part_l, a.part_o, (int)RH, (int)H, (int)L,
                           a.pos, clat);
    else if (a.nslice <= 2 * kCombineSmallSlices)
        hipLaunchKernelGGL((k_mla_combine_mfma<2 * kCombineSmallSlices, 1024>), cgrid, dim3(1024), 0,
                           ctx->stream, a.part_m, a.part_l, a.part_o, (int)RH, (int)H, (int)L,
                           a.pos, clat);
    else
        hipLaunchKernelGGL((k_mla_combine_mfma<kMlaMaxSlices, 1024>), cgrid, dim3(1024), 0,
                           ctx->stream, a.part_m, a.part_l, a.part_o, (int)RH, (int)H, (int)L,
                           a.pos, clat);
    timing_end(ctx, tok);
    return launch_check(ctx, "k_mla_combine_mfma");
}

int32_t launch_mla_attend(ut_ctx *ctx, const float *qabs, const float *qrope, const float *latent,
                          const float *krot, int64_t R, int64_t H, int64_t L, int64_t P,
                          int64_t pos_base, float scale, float *clat, void *scratch) {
    const int64_t T = pos_extent(ctx, pos_base + R);  // positions any row can see
    if (mla_mfma_ok(H, L, P, T)) {
        // the f32 cache is split into the MFMA form in scratch first
        __bf16 *kc = (__bf16 *)((char *)scratch + mla_mfma_scratch_bytes(R, H, L, T));
        UT_TRY(launch_mla_cache_split(ctx, latent, krot, T, L, P, kc));
        return launch_mla_attend_kc(ctx, qabs, qrope, kc, R, H, L, P, pos_base, scale, clat,
                                    scratch);
    }
    const int nsplit = (int)((T + kMlaSlice - 1) / kMlaSlice);
    const size_t n = (size_t)R * H * nsplit;
    float *pm = (float *)scratch;
    float *pl = (float *)((char *)scratch + ((n * 4 + 255) & ~size_t(255)));
    float *po = (float *)((char *)pl + ((n * 4 + 255) & ~size_t(255)));
    if (L % 4 != 0) {
        set_error(ctx, "mla: latent width %lld must be a multiple of 4", (long long)L);
        return UT_ERR_SHAPE;
    }
    int HG = 8;
    while (HG > 1 && H % HG != 0) HG >>= 1;
    const size_t shmem = (size_t)HG * (L + P + kMlaSlice) * 4;
    if (shmem > 64 * 1024) {
        set_error(ctx, "mla: L + P too large for the LDS staging (%lld)", (long long)(L + P));
        return UT_ERR_SHAPE;
    }
    dim3 grid((unsigned)(R * H / HG), (unsigned)nsplit);
    const PosRef pr = pos_ref(ctx, pos_base);
    int tok = timing_begin(ctx, "mla_split");
    switch (HG) {
    case 8: hipLaunchKernelGGL(k_mla_split<8>, grid, dim3(256), shmem, ctx->stream, qabs, qrope, latent, krot, (int)R, (int)H, (int)L, (int)P, pr, scale, pm, pl, po, nsplit); break;
    case 4: hipLaunchKernelGGL(k_mla_split<4>, grid, dim3(256), shmem, ctx->stream, qabs, qrope, latent, krot, (int)R, (int)H, (int)L, (int)P, pr, scale, pm, pl, po, nsplit); break;
    case 2: hipLaunchKernelGGL(k_mla_split<2>, grid, dim3(256), shmem, ctx->stream, qabs, qrope, latent, krot, (int)R, (int)H, (int)L, (int)P, pr, scale, pm, pl, po, nsplit); break;
    default: hipLaunchKernelGGL(k_mla_split<1>, grid, dim3(256), shmem, ctx->stream, qabs, qrope, latent, krot, (int)R, (int)H, (int)L, (int)P, pr, scale, pm, pl, po, nsplit); break;
    }
    timing_end(ctx, tok);
    UT_TRY(launch_check(ctx, "k_mla_split"));
    tok = timing_begin(ctx, "mla_combine");
    hipLaunchKernelGGL(k_mla_combine, dim3((unsigned)(R * H)), dim3(256), 0, ctx->stream, pm, pl,
                       po, (int)L, (int)H, pr, nsplit, clat);
    timing_end(ctx, tok);
    return launch_check(ctx, "k_mla_combine");
}

}  // namespace ut

using namespace ut;

extern "C" int32_t ut_mla_attend(ut_ctx *ctx, const float *qabs_dev, const float *q_rope_dev,
                                 const float *latent_dev, const float *krot_dev, int64_t R,
                                 int64_t H, int64_t L, int64_t P, int64_t pos_base, float scale,
                                 float *clat_dev) {
    if (!ctx || !qabs_dev || !latent_dev || !clat_dev || R <= 0 || H <= 0 || L <= 0 || P < 0 ||
        pos_base < 0 || (P > 0 && (!q_rope_dev || !krot_dev))) {
        set_error(ctx, "ut_mla_attend: bad argument");
        return UT_ERR_ARG;
    }
    ScratchPlan plan;
    plan.add(mla_scratch_bytes(R, H, L, P, pos_base + R));
    std::vector<void *> ptrs;
    UT_TRY(scratch_acquire(ctx, plan, ptrs));
    return launch_mla_attend(ctx, qabs_dev, q_rope_dev, latent_dev, krot_dev, R, H, L, P, pos_base,
                             scale, clat_dev, ptrs[0]);
}

extern "C" int32_t ut_mla_cache_split(ut_ctx *ctx, const float *latent_dev, const float *krot_dev,
                                      int64_t T, int64_t L, int64_t P, void *kc_dev) {
    if (!ctx || !latent_dev || !krot_dev || !kc_dev || T < 0 || L <= 0 || P <= 0) {
        set_error(ctx, "ut_mla_cache_split: bad argument");
        return UT_ERR_ARG;
    }
    if (((uintptr_t)kc_dev & 15) != 0) {
        set_error(ctx, "ut_mla_cache_split: kc must be 16-byte aligned");
        return UT_ERR_ARG;
    }
    return launch_mla_cache_split(ctx, latent_dev, krot_dev, T, L, P, (__bf16 *)kc_dev);
}

extern "C" int32_t ut_mla_attend_split(ut_ctx *ctx, const float *qabs_dev, const float *q_rope_dev,
                                       const void *kc_dev, int64_t R, int64_t H, int64_t L,
                                       int64_t P, int64_t pos_base, float scale, float *clat_dev) {
    if (!ctx || !qabs_dev || !q_rope_dev || !kc_dev || !clat_dev || R <= 0 || H <= 0 || L <= 0 ||
        P <= 0 || pos_base < 0) {
        set_error(ctx, "ut_mla_attend_split: bad argument");
        return UT_ERR_ARG;
    }
    if (!mla_kc_ok(H, L, P, pos_base + R)) {
        set_error(ctx, "ut_mla_attend_split: shape (H %lld, L %lld, P %lld, T %lld) not supported",
                  (long long)H, (long long)L, (long long)P, (long long)(pos_base + R));
        return UT_ERR_SHAPE;
    }
    ScratchPlan plan;
    plan.add(mla_kc_scratch_bytes(R, H, L, pos_base + R));
    std::vector<void *> ptrs;
    UT_TRY(scratch_acquire(ctx, plan, ptrs));
    return launch_mla_attend_kc(ctx, qabs_dev, q_rope_dev, (const __bf16 *)kc_dev, R, H, L, P,
                                pos_base, scale, clat_dev, ptrs[0]);
}
