// ut_mla.h -- internal interface of the MLA attention kernels.
#pragma once

#include "ut_internal.h"

namespace ut {

// Scratch bytes of launch_mla_attend for R rows over T positions.
size_t mla_scratch_bytes(int64_t R, int64_t H, int64_t L, int64_t P, int64_t T);
// The MFMA path over a cache kept in split form: per position the bf16 hi
// parts of [latent | k_rot] then the lo parts (2 * (L + P) bf16, the bytes
// of the f32 cache).  Taken for 32k heads, latent 512 and rope 64, up to a
// context length T whose slice count fits the combine.
bool mla_kc_ok(int64_t H, int64_t L, int64_t P, int64_t T);
size_t mla_kc_scratch_bytes(int64_t R, int64_t H, int64_t L, int64_t T);
int32_t launch_mla_cache_split(ut_ctx *ctx, const float *latent, const float *krot, int64_t T,
                               int64_t L, int64_t P, __bf16 *kc);
int32_t launch_mla_attend_kc(ut_ctx *ctx, const float *qabs, const float *qrope, const __bf16 *kc,
                             int64_t R, int64_t H, int64_t L, int64_t P, int64_t pos_base,
                             float scale, float *clat, void *scratch);
int32_t launch_mla_attend(ut_ctx *ctx, const float *qabs, const float *qrope, const float *latent,
                          const float *krot, int64_t R, int64_t H, int64_t L, int64_t P,
                          int64_t pos_base, float scale, float *clat, void *scratch);

}  // namespace ut
