// ut_sample.h -- internal interface of the argmax kernels.
#pragma once

#include "ut_argmax.h"
#include "ut_internal.h"

namespace ut {

int64_t argmax_parts(int64_t V);
size_t argmax_scratch_bytes(int64_t rows, int64_t V);
// The most partials per row a GEMV epilogue over V output rows leaves.
int64_t argmax_gemv_parts_max(int64_t V);
// Partials of rows rows at stride in the argmax scratch.
ArgmaxParts argmax_parts_view(void *scratch, int64_t rows, int64_t stride);
// idx [rows] (device) = argmax of each row of x [rows, ldx] over V columns.
// err (optional): the sticky error word, copied to idx[rows]; with it, tail
// (optional, ntail <= 256 ints) is copied to idx[rows + 1 ...].
int32_t launch_argmax(ut_ctx *ctx, const float *x, int64_t rows, int64_t V, int64_t ldx,
                      int32_t *idx, void *scratch, const int32_t *err = nullptr,
                      const int32_t *tail = nullptr, int ntail = 0);
// The same from partials a GEMV epilogue left (p.stride per row).
int32_t launch_argmax_final(ut_ctx *ctx, const float *x, int64_t rows, int64_t ldx,
                            const ArgmaxParts &p, int32_t *idx, const int32_t *err = nullptr,
                            const int32_t *tail = nullptr, int ntail = 0);

}  // namespace ut
