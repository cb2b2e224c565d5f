// ut_internal.h -- shared host/device definitions of the gfx950 backend.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

#include "../../include/undertow_hip.h"

namespace ut {

// ------------------------------------------------------------- errors ---
// Failures are reported as status codes; the message is kept on the ctx.
void set_error(ut_ctx *ctx, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

#define UT_CHECK_HIP(ctx, expr)                                                     \
    do {                                                                            \
        hipError_t e_ = (expr);                                                     \
        if (e_ != hipSuccess) {                                                     \
            ::ut::set_error((ctx), "%s failed: %s (%s:%d)", #expr,                 \
                            hipGetErrorString(e_), __FILE__, __LINE__);             \
            return UT_ERR_HIP;                                                      \
        }                                                                           \
    } while (0)

#define UT_TRY(expr)                    \
    do {                                \
        int32_t rc_ = (expr);           \
        if (rc_ != UT_OK) return rc_;   \
    } while (0)

// ------------------------------------------------------------ context ---
struct KernelStat {
    std::string name;
    int64_t launches = 0;
    double total_ms = 0.0;
};

struct PendingTiming {
    int stat;
    hipEvent_t start, stop;
};

struct DeviceBuffer {
    void *ptr = nullptr;
    size_t bytes = 0;
};

}  // namespace ut

struct ut_ctx {
    int device = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    std::string err;
    // Scratch arena: one device allocation, carved per call.  All work runs
    // on one stream, so a later call may reuse what an earlier one used.
    ut::DeviceBuffer scratch;
    // Pinned host staging for small device->host results.
    void *pinned = nullptr;
    size_t pinned_bytes = 0;
    // Kernel timing (bench tooling).
    bool timing = false;
    std::vector<ut::KernelStat> stats;
    std::vector<ut::PendingTiming> pending;
    int multiprocessors = 256;
    // Sticky device-side error flag (invalid expert ids), reported by the
    // next ut_ctx_synchronize().
    int32_t *dev_err = nullptr;
    // Split-K GEMV partial totals (allocated on first use).
    void *splitk = nullptr;
    // Device address of this device's copy of the expert block's fixed
    // working array (ut_moe_experts_noalloc), from hipGetSymbolAddress at
    // context creation.
    void *noalloc_scratch = nullptr;
    // The opt-in fast-int8 matmul (ut_set_fast_int8): off by default.
    bool fast_int8 = false;
    // While a session captures its decode step into a graph: the device word
    // holding the step's position, the host position it held at capture
    // (positions passed to launchers are taken relative to it) and the
    // session's capacity (grids that depend on the context length are sized
    // for it).  step_pos == nullptr: positions are host values.
    const int64_t *step_pos = nullptr;
    int64_t step_pos_host = 0, step_cap = 0;
    // Handle lifetime: models hold a reference on their context and
    // sessions on their model, so the handles may be released in any order.
    int refs = 1;
};

namespace ut {
// A position handed to a kernel: a host value, or (in a captured decode
// step) an offset from a device word read when the kernel runs, so each
// replay of the step sees the session's current position.
struct PosRef {
    int64_t base = 0;
    const int64_t *dev = nullptr;
    __device__ __forceinline__ int64_t get() const { return dev ? base + *dev : base; }
};
inline PosRef pos_ref(const ut_ctx *ctx, int64_t pos) {
    PosRef r;
    if (ctx->step_pos) {
        r.base = pos - ctx->step_pos_host;
        r.dev = ctx->step_pos;
    } else {
        r.base = pos;
    }
    return r;
}
// The positions a launch can see at most: pos_end itself, or the capacity
// while a decode step is captured.
inline int64_t pos_extent(const ut_ctx *ctx, int64_t pos_end) {
    return ctx->step_pos ? ctx->step_cap : pos_end;
}
}  // namespace ut

struct ut_qtensor {
    int32_t fmt = UT_FMT_F32;
    int64_t out_dim = 0, in_dim = 0;
    int64_t row_bytes = 0;     // payload bytes per output row
    void *payload = nullptr;   // device
    float *scales = nullptr;   // device, out_dim floats (int formats)
    bool owns = true;          // false: views into a model arena
    int device = 0;
};

namespace ut {

// Scratch carving: returns device pointers into ctx->scratch, growing it
// (after a stream sync) when needed.  Each carve is 256-byte aligned.
struct ScratchPlan {
    std::vector<size_t> sizes;
    size_t add(size_t bytes) {
        sizes.push_back((bytes + 255) & ~size_t(255));
        return sizes.size() - 1;
    }
};
int32_t scratch_acquire(ut_ctx *ctx, const ScratchPlan &plan, std::vector<void *> &ptrs);
int32_t pinned_acquire(ut_ctx *ctx, size_t bytes, void **ptr);

// Kernel timing hooks: call timing_begin before a launch and timing_end
// after it; both are no-ops unless timing is enabled on the ctx.
int timing_begin(ut_ctx *ctx, const char *name);
void timing_end(ut_ctx *ctx, int token);
int32_t launch_check(ut_ctx *ctx, const char *name);
void ctx_retain(ut_ctx *ctx);
void ctx_release(ut_ctx *ctx);
// The context's device error flag (allocated when the context is created)
// and its check.
int32_t device_error_flag(ut_ctx *ctx, int32_t **flag);
// Looks up this device's copy of the expert block's fixed working array
// (hipGetSymbolAddress, the device current) into ctx->noalloc_scratch.
int32_t moe_noalloc_scratch_init(ut_ctx *ctx);
// Gives up the context's claim on its device's working array (at destroy).
void moe_noalloc_release(const ut_ctx *ctx);
// Split-K partials buffer of the context (kSplitKPartBytes), allocated on
// first use: four rows of the LM head's logits (129,280) over four splits.
constexpr int64_t kSplitKPartBytes = int64_t(32) << 20;
int32_t splitk_buffer(ut_ctx *ctx, int64_t **part);
int32_t check_device_error(ut_ctx *ctx);

int64_t payload_bytes(int32_t fmt, int64_t out_dim, int64_t in_dim);

// ---------------------------------------------------- activation digits ---
// Integer form of an f32 activation row used by the quantized GEMVs:
//   x~[k] = rint(x[k] * 2^(22 - E)),  E = exponent with max|x| < 2^E,
// so |x~| <= 2^22.  The quantized products then accumulate exactly in
// integers: S = sum_k x~[k] q[k], and out = fl(fl(S * 2^(E-22)) * scale).
// The same S results for any tiling, reduction order or row count.
//
// Layout of one digitised batch (rows m < M, K columns, K8 = ceil(K/8),
// K4 = ceil(K/4)):
//   exps  [M]            int32: E - 22 (INT32_MIN when the row is non-finite)
//   dig4  [M][6][K8]     uint32: balanced base-16 digits d_p in [-8,7] of x~,
//                        nibble j of word c8 = digit of column 8*c8 + j
//   dig8  [M][3][K4]     uint32: balanced base-256 digits in [-128,127],
//                        byte j of word c4 = digit of column 4*c4 + j
//   xt    [M][K]         int32: x~ itself (generic kernels)
struct XDigits {
    int32_t *exps = nullptr;
    uint32_t *dig4 = nullptr;
    uint32_t *dig8 = nullptr;
    int32_t *xt = nullptr;
    int64_t M = 0, K = 0;
};
enum { XD_DIG4 = 1, XD_DIG8 = 2, XD_XT = 4 };
size_t xdigits_bytes(int64_t M, int64_t K, int flags);
// The rows s0.. of a digitised batch.
inline XDigits xdigits_rows(const XDigits &d, int64_t s0) {
    XDigits r = d;
    const int64_t K8 = (d.K + 7) / 8, K4 = (d.K + 3) / 4;
    r.exps = d.exps ? d.exps + s0 : nullptr;
    r.dig4 = d.dig4 ? d.dig4 + s0 * 6 * K8 : nullptr;
    r.dig8 = d.dig8 ? d.dig8 + s0 * 3 * K4 : nullptr;
    r.xt = d.xt ? d.xt + s0 * d.K : nullptr;
    r.M = d.M - s0;
    return r;
}
// Carves an XDigits view out of `base` (device memory of xdigits_bytes()).
XDigits xdigits_view(void *base, int64_t M, int64_t K, int flags);
// Digitise x [M, K] (row stride ldx floats).  rowmax_bits: optional
// precomputed max|x| per row (float bits, as atomicMax'd by a producer).
int32_t launch_digitize(ut_ctx *ctx, const float *x, int64_t ldx, int64_t M, int64_t K,
                        const uint32_t *rowmax_bits, XDigits xd, int flags);
// Same with the row maxima given as nparts partial maxima per row
// ([M][nparts] float bits), reduced by the kernel.
int32_t launch_digitize_parts(ut_ctx *ctx, const float *x, int64_t ldx, int64_t M, int64_t K,
                              const uint32_t *rowmax_parts, int32_t nparts, XDigits xd,
                              int flags);

// rmsnorm (undertow-quant/src/lib.rs:91-100) of each row fused with its
// digitisation; out (optional) receives the normalised f32 row.
int32_t launch_rmsnorm_digitize(ut_ctx *ctx, const float *x, int64_t ldx, int64_t M, int64_t K,
                                const float *w, float eps, float *out, int64_t ldo, XDigits xd,
                                int flags);

// Flags a GEMV needs for a weight of this format and shape.
int xdigit_flags_for(int32_t fmt, int64_t K);

// ---------------------------------------------------------- GEMV core ---
// out[m, o] (row stride ldo) for one quantized matrix, all rows o < O.
// x is given digitised (int formats) or as f32 (fmt F32).
// Split-K partials handed to the consumer instead of a sum launch: ks > 1
// means part[z][M][O] holds int64 totals (f32 weights: the float's bits)
// that the consumer sums in z order; ks == 1 means out was written.
struct SplitKPartials {
    int64_t *part = nullptr;
    int ks = 1;
    int64_t O = 0;
};

// A kv_a row's cache append (kv_append_row) run by one workgroup of
// another launch: comp = the finished [L + P] row.
struct KvAppendArgs {
    const float *comp = nullptr;  // nullptr: none
    int64_t L = 0, P = 0;
    const float *w = nullptr;
    float eps = 0.0f;
    float *latent = nullptr, *krot = nullptr;
    __bf16 *kc = nullptr;
    PosRef pos;
    const float2 *table = nullptr;
};

// A GEMV epilogue's argmax partials (ut_argmax.h): workgroup j of the
// producing launch writes the best (value, row) of activation row m among
// the output rows it finished to v[m * stride + j], i[m * stride + j].
struct ArgmaxParts {
    float *v = nullptr;  // nullptr: no partials
    int32_t *i = nullptr;
    int64_t stride = 0;
};

struct GemvArgs {
    const ut_qtensor *w = nullptr;
    const float *xf = nullptr;  // f32 activations [M, K] (F32 weights)
    XDigits xd;                 // digitised activations (int weights)
    int64_t M = 0;
    float *out = nullptr;
    int64_t ldo = 0;
    int accumulate = 0;         // out += result instead of out = result
    // optional second weight (same format, K and row bytes) -> out2[M, ldo2]
    const ut_qtensor *w2 = nullptr;
    float *out2 = nullptr;
    int64_t ldo2 = 0;
    // optional: leave split-K partials to the consumer (M <= 4, fast path)
    SplitKPartials *defer = nullptr;
    // optional (int weights, fast path): digitise xf while staging, with the
    // row shift from partial maxima of |x| (float bits, [M][nxmax]) written
    // by the producer; the rows' exponents go to exps_out [M]
    const uint32_t *xmax = nullptr;
    int nxmax = 0;
    int32_t *exps_out = nullptr;
    // optional (M <= 4, one weight, no defer): when the GEMV splits K, its
    // partial sum also runs this rmsnorm+digitise on the finished rows (one
    // launch instead of two); *next_done reports whether it did
    const struct NormNext *next = nullptr;
    bool *next_done = nullptr;
    // optional (M <= 4, one weight, no defer, no next): the launch that
    // finishes the output rows also leaves argmax partials per workgroup in
    // am_scratch (argmax_scratch_bytes) and reports their view in *am_out
    // (am_out->v == nullptr: it did not)
    void *am_scratch = nullptr;
    ArgmaxParts *am_out = nullptr;
    // optional (one row; gemv_norm_ok): xf is the un-normalised row, which
    // the GEMV rms-normalises with norm_w (eps norm_eps) and digitises while
    // staging it, with the row digitiser's arithmetic, so the outputs equal
    // the GEMV of that digitiser's digits bit for bit
    const float *norm_w = nullptr;
    float norm_eps = 0.0f;
    // optional with norm_w: the launch also appends this kv_a row
    const KvAppendArgs *kv = nullptr;
};
bool gemv_norm_ok(const ut_qtensor *w, int64_t M, const void *x, const void *norm_w);
// The embedding lookup (launch_embed) and the norm that follows it
// (rmsnorm + digits as NormNext asks) in one launch; x gets the looked-up
// rows.  embed_norm_ok: rows of K % 8 == 0 columns, K <= 8192, aligned.
struct NormNext;
// The MTP module's input rows [enorm(embed(ids)) | hnorm(hidden)] into
// cat [rows][2H] in one launch, with each half's max|v| in vmax [rows][2]
// (float bits) for a GEMV that digitises cat while staging it
// (GemvArgs::xmax, nxmax = 2).
bool mtp_input_ok(int64_t H);
int32_t launch_mtp_input(ut_ctx *ctx, const ut_qtensor *emb, const int32_t *ids,
                         const float *hidden, int64_t rows, int64_t H, const float *enorm,
                         const float *hnorm, float eps, float *cat, uint32_t *vmax);
bool embed_norm_ok(const ut_qtensor *emb, int64_t K, const float *x, const float *norm_w);
int32_t launch_embed_norm(ut_ctx *ctx, const ut_qtensor *emb, const int32_t *ids, int64_t rows,
                          float *x, int64_t ldx, const NormNext &nx);
// One row of an int8 weight (or the w/w2 pair) with every row finished in
// its workgroup (K split inside it): no partials.  Checks gemv_rowsplit_ok.
bool gemv_rowsplit_ok(const GemvArgs &ga);
int32_t launch_gemv_rowsplit(ut_ctx *ctx, const GemvArgs &ga);
int32_t gemv(ut_ctx *ctx, const GemvArgs &a);
// The kv_a / q_a pair GEMV's deferred split-K partials (kv_a rows first)
// finished in one launch: q_a rows rms-normalised into qa_n and digitised
// into qd (flags), kv_a rows appended to the cache (as launch_kv_append).
// qa_raw set: q_a rows are only summed, into qa_raw, for a consumer that
// normalises them itself (GemvArgs::norm_w).
constexpr int64_t kMlaPreMaxComp = 1024;  // kv_lora_rank + qk_rope_head_dim bound
bool mla_pre_ok(int64_t M, int64_t q_lora, int64_t L, int64_t P);
int32_t launch_mla_pre(ut_ctx *ctx, const SplitKPartials &pp, int64_t O1, const int32_t *exps,
                       const float *kv_scales, const float *q_scales, int64_t M, int64_t q_lora,
                       const float *q_norm, float eps, float *qa_n, const XDigits &qd, int flags,
                       int64_t L, int64_t P, const float *kv_norm, float *latent, float *krot,
                       __bf16 *kc, int64_t pos_base, const float2 *table,
                       float *qa_raw = nullptr);
// f32 weights, M <= 4 rows, out [M][ldo]: one workgroup per output row
bool rowdot_f32_ok(const ut_qtensor *w, int64_t M);
int32_t launch_rowdot_f32(ut_ctx *ctx, const ut_qtensor *w, const float *x, int64_t M,
                          float *out, int64_t ldo);
// Whether the fast (digit / vector) GEMV takes this weight.
bool gemv_fast_ok(const ut_qtensor *w);

// out[M, ldo] (+)= x[M, K] * w^T with x f32 on device: digitises x into
// digit_scratch (matmul_digit_bytes(M, K) bytes) when w is quantized.
size_t matmul_digit_bytes(int64_t M, int64_t K);
// Same with x already digitised (xd must hold the form the weight needs;
// x is read only for f32 weights).
int32_t matmul_digits(ut_ctx *ctx, const ut_qtensor *w, const float *x, const XDigits &xd,
                      int64_t M, float *out, int64_t ldo, int accumulate);
// matmul_digits into out [M][out_dim], then idx [M] = each row's argmax;
// the GEMV that finishes the rows leaves the argmax partials where it can
// (am_scratch: argmax_scratch_bytes(M, out_dim)); err: the sticky error word
// copied to idx[M], and with it ntail ints of tail to idx[M + 1 ...].
int32_t matmul_digits_argmax(ut_ctx *ctx, const ut_qtensor *w, const float *x, const XDigits &xd,
                             int64_t M, float *out, int32_t *idx, void *am_scratch,
                             const int32_t *err, const int32_t *tail = nullptr, int ntail = 0);
int32_t matmul_dev(ut_ctx *ctx, const ut_qtensor *w, const float *x, int64_t M, float *out,
                   int64_t ldo, int accumulate, void *digit_scratch);

}  // namespace ut
