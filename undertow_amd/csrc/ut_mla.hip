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
                                                   int L, int P, int64_t pos_base, float scale,
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
    const int64_t n_ctx = pos_base + r + 1;
    const int64_t t0 = (int64_t)j * kMlaSlice;
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
                                                     int H, int64_t pos_base, int nsplit,
                                                     float *__restrict__ clat) {
    const int64_t qi = blockIdx.x;  // r*H + h
    const int r = (int)(qi / H);
    const int64_t n_ctx = pos_base + r + 1;
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

size_t mla_scratch_bytes(int64_t R, int64_t H, int64_t L, int64_t T) {
    int64_t ns = (T + kMlaSlice - 1) / kMlaSlice;
    size_t n = (size_t)R * H * ns;
    return ((n * 4 + 255) & ~size_t(255)) * 2 + ((n * L * 4 + 255) & ~size_t(255));
}

int32_t launch_mla_attend(ut_ctx *ctx, const float *qabs, const float *qrope, const float *latent,
                          const float *krot, int64_t R, int64_t H, int64_t L, int64_t P,
                          int64_t pos_base, float scale, float *clat, void *scratch) {
    const int64_t T = pos_base + R;  // positions any row can see
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
    int tok = timing_begin(ctx, "mla_split");
    switch (HG) {
    case 8: hipLaunchKernelGGL(k_mla_split<8>, grid, dim3(256), shmem, ctx->stream, qabs, qrope, latent, krot, (int)R, (int)H, (int)L, (int)P, pos_base, scale, pm, pl, po, nsplit); break;
    case 4: hipLaunchKernelGGL(k_mla_split<4>, grid, dim3(256), shmem, ctx->stream, qabs, qrope, latent, krot, (int)R, (int)H, (int)L, (int)P, pos_base, scale, pm, pl, po, nsplit); break;
    case 2: hipLaunchKernelGGL(k_mla_split<2>, grid, dim3(256), shmem, ctx->stream, qabs, qrope, latent, krot, (int)R, (int)H, (int)L, (int)P, pos_base, scale, pm, pl, po, nsplit); break;
    default: hipLaunchKernelGGL(k_mla_split<1>, grid, dim3(256), shmem, ctx->stream, qabs, qrope, latent, krot, (int)R, (int)H, (int)L, (int)P, pos_base, scale, pm, pl, po, nsplit); break;
    }
    timing_end(ctx, tok);
    UT_TRY(launch_check(ctx, "k_mla_split"));
    tok = timing_begin(ctx, "mla_combine");
    hipLaunchKernelGGL(k_mla_combine, dim3((unsigned)(R * H)), dim3(256), 0, ctx->stream, pm, pl,
                       po, (int)L, (int)H, pos_base, nsplit, clat);
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
    plan.add(mla_scratch_bytes(R, H, L, pos_base + R));
    std::vector<void *> ptrs;
    UT_TRY(scratch_acquire(ctx, plan, ptrs));
    return launch_mla_attend(ctx, qabs_dev, q_rope_dev, latent_dev, krot_dev, R, H, L, P, pos_base,
                             scale, clat_dev, ptrs[0]);
}
