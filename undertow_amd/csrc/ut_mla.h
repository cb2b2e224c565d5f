// ut_mla.h -- internal interface of the MLA attention kernels.
#pragma once

#include "ut_internal.h"

namespace ut {

// Scratch bytes of launch_mla_attend for R rows over T positions.
size_t mla_scratch_bytes(int64_t R, int64_t H, int64_t L, int64_t P, int64_t T);
int32_t launch_mla_attend(ut_ctx *ctx, const float *qabs, const float *qrope, const float *latent,
                          const float *krot, int64_t R, int64_t H, int64_t L, int64_t P,
                          int64_t pos_base, float scale, float *clat, void *scratch);

}  // namespace ut
