// ut_ops.h -- the small per-layer kernels of the decode step.
#pragma once

#include "ut_internal.h"

namespace ut {

// Embedding rows (model.rs:119-122): out[s] = 0 + (1*scale[id])*q[id] (f32
// tables copied).  ids: device int32 [rows].
int32_t launch_embed(ut_ctx *ctx, const ut_qtensor *emb, const int32_t *ids, int64_t rows,
                     float *out, int64_t ldo);
// rmsnorm (undertow-quant/src/lib.rs:91-100) per row: the mean of squares in
// f64, r = 1/sqrt((float)ms + eps), out = (x*r)*w.
int32_t launch_rmsnorm(ut_ctx *ctx, const float *x, int64_t ldx, const float *w, int64_t n,
                       float eps, int64_t rows, float *out, int64_t ldo);
// rope_interleave (attention.rs:106-118) in place on `heads` slices of
// `dim` floats per row: slice (s, h) at v + s*ld_row + h*ld_head, position
// pos_base + s.  table: [positions][dim/2] (cos, sin) computed on the host.
int32_t launch_rope(ut_ctx *ctx, float *v, int64_t rows, int64_t heads, int64_t ld_row,
                    int64_t ld_head, int64_t dim, int64_t pos_base, const float2 *table,
                    int64_t table_stride);
// y += x (f32 adds), n elements.
int32_t launch_add(ut_ctx *ctx, float *y, const float *x, int64_t n);
// Absorbed query (attention.rs:204-213): for each (s, h)
//   qabs[s,h,:] = sum_d (q[s,h,d]*scale[h*kvh+d]) * W[h*kvh+d, :]  (d < nope,
//   adds in d order) and q_rope[s,h,:] = rope_interleave(q[s,h,nope:], pos_base+s).
int32_t launch_absorb_q(ut_ctx *ctx, const ut_qtensor *kv_b, const float *q, int64_t rows,
                        int64_t heads, int64_t nope, int64_t rope, int64_t vh, float *qabs,
                        float *qrope, int64_t pos_base, const float2 *table);
// Cache append (attention.rs:168-186) for rows at positions pos_base..:
// latent = rmsnorm(comp[:L], w), krot = rope_interleave(comp[L:L+P], pos),
// stored as f32 (latent, krot) or, with kc, in the MFMA attention's split
// bf16 form (per position: hi parts of [latent | krot], then lo parts).
int32_t launch_kv_append(ut_ctx *ctx, const float *comp, int64_t rows, int64_t L, int64_t P,
                         const float *w, float eps, float *latent, float *krot, __bf16 *kc,
                         int64_t pos_base, const float2 *table);
// Absorbed value (attention.rs:235, QTensor::matvec_rows): for each (s, h)
//   ctx[s, h*vh + j] = (sum_i clat[s,h,i] * W[h*kvh+nope+j, i]) * scale.
int32_t launch_absorb_v(ut_ctx *ctx, const ut_qtensor *kv_b, const float *clat, int64_t rows,
                        int64_t heads, int64_t nope, int64_t vh, float *out);

}  // namespace ut
