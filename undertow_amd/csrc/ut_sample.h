// ut_sample.h -- internal interface of the argmax kernels.
#pragma once

#include "ut_internal.h"

namespace ut {

int64_t argmax_parts(int64_t V);
size_t argmax_scratch_bytes(int64_t rows, int64_t V);
// idx [rows] (device) = argmax of each row of x [rows, ldx] over V columns.
int32_t launch_argmax(ut_ctx *ctx, const float *x, int64_t rows, int64_t V, int64_t ldx,
                      int32_t *idx, void *scratch);

}  // namespace ut
