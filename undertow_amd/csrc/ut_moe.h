// ut_moe.h -- internal interface of the expert block and router kernels.
#pragma once

#include "ut_internal.h"

namespace ut {

constexpr int kGateUpRowsPerWG = 16;  // h rows per gate/up workgroup
constexpr int kDownMaxSplit = 16;     // K splits of a one-slot MLP's down projection

// Device arrays of per-expert pointers (indexed by expert id).
struct ExpertPtrs {
    const uint8_t *const *gate_w = nullptr;
    const uint8_t *const *up_w = nullptr;
    const uint8_t *const *down_w = nullptr;
    const float *const *gate_s = nullptr;
    const float *const *up_s = nullptr;
    const float *const *down_s = nullptr;
};

struct MoePlan {
    int32_t *count;        // number of slots used
    int32_t *uniq;         // [slots] expert id per slot
    int32_t *choice_slot;  // [M*k] slot of each (row, choice), -1 when invalid
    // [slots][6] the slot's weight pointers (gate, up, down payloads, then
    // their scales), resolved once so the expert kernels start with a
    // single dependent load
    const void **sp;
};

// Pointer i (0..5: gate, up, down payloads; gate, up, down scales) of
// expert e in a [6][E] device pointer table.
enum { kSpGate = 0, kSpUp = 1, kSpDown = 2, kSpGateS = 3, kSpUpS = 4, kSpDownS = 5 };

// One pass of the expert block over M <= 4 rows (all on device).
// The next input norm, run by the launch that finishes a residual row:
// normed = rmsnorm(out row, norm_w) (f32, row stride ldn) and its digit
// forms (flags) in nd, rows counted from the call's first row.
struct NormNext {
    const float *norm_w = nullptr;
    float eps = 0.0f;
    float *normed = nullptr;
    int64_t ldn = 0;
    XDigits nd;
    int flags = 0;
    // optional: the finished (un-normalised) rows also go to raw2 at rows
    // pos2, pos2 + 1, ... (stride ld2): the MTP head's hidden-state rows
    float *raw2 = nullptr;
    int64_t ld2 = 0;
    PosRef pos2;
};

struct MoeCall {
    int fmt = UT_FMT_INT4;
    ExpertPtrs tbl;
    int64_t E = 0, H = 0, I = 0;
    int M = 1, k = 1;
    const int32_t *ids = nullptr;      // [M, k]
    const float *weights = nullptr;    // [M, k]
    const float *x = nullptr;          // [M, H]
    const uint16_t *xh = nullptr;      // [M, H] bf16 activations in place of x
    const XDigits *x_digits = nullptr; // optional: x already digitised
    float *out = nullptr;              // [M, ldo]
    int64_t ldo = 0;
    int accumulate = 0;
    int extra_slot = -1;  // >= 0: expert id always appended as the last slot, added with weight 1
    int32_t *err_flag = nullptr;
    bool plan_ready = false;  // the slot plan is already in the scratch (launch_route_plan)
    // x (f32) holds exactly the values x_digits were made from (the
    // matrix-core expert kernels then stage x themselves)
    bool x_matches_digits = false;
    const MoePlan *plan = nullptr;  // a fixed plan elsewhere (one-slot MLPs)
    const float *init = nullptr;    // combine starts from init[M, ldo] instead of zero
    // Optional one-slot MLP (a shared expert, format int4 or int8 like the
    // routed experts) run in the same gate/up and down launches as the
    // routed experts and added after the routed sum.  Its fmt, tbl, I and
    // plan are used; it needs x_digits holding both formats' digits and its
    // own scratch of moe_layout(M, 1, 1, H, I, fmt).total bytes.
    const MoeCall *shared = nullptr;
    void *shared_scratch = nullptr;
    // optional: the combine also rms-normalises and digitises the finished
    // rows of out (one launch instead of two; H <= 8192, H % 8 == 0)
    const NormNext *next = nullptr;
    // optional: route too (k_route_wave's semantics) from the router logits
    // [M, E]; the choices land in route_ids / route_w (which ids / weights
    // must name).  Done inside the gate/up launch where it can be, else by a
    // route launch first.
    const float *route_logits = nullptr;
    const float *route_bias = nullptr;
    int route_ng = 1, route_tg = 1, route_norm = 0;
    float route_scale = 1.0f;
    int32_t *route_ids = nullptr;
    float *route_w = nullptr;
};
bool moe_combine_norm_ok(int64_t H);
// The fewest rows that take the int8 experts' matrix-core kernels (config
// 2's int8 variant per step: two rows 4,760 -> 5,362 GB/s, four rows
// 3,519 -> 5,321 GB/s against the dot-product kernels; one row stays on
// those, 5,296 GB/s).
#ifndef UT_MOE_I8_MFMA_MIN_M
#define UT_MOE_I8_MFMA_MIN_M 2
#endif
// Whether the matrix-core gate/up takes an expert pass of M rows (int4:
// 2..4 rows, hidden a multiple of 512; int8: UT_MOE_I8_MFMA_MIN_M..4 rows,
// hidden a multiple of 256).
inline bool gate_up_mfma_ok(int fmt, int M, int64_t H) {
    if (fmt == UT_FMT_INT8) return M >= UT_MOE_I8_MFMA_MIN_M && M <= 4 && H % 256 == 0;
    return fmt == UT_FMT_INT4 && M >= 2 && M <= 4 && H % 512 == 0;
}

struct ScratchLayout {
    size_t total = 0;
    size_t count = 0, uniq = 0, choice = 0, sp = 0, xd = 0, h = 0, hmax = 0, hd = 0, d = 0, dpart = 0;
    size_t xw = 0;  // bf16 activations widened to f32 (when not staged by gate/up)
    size_t arrive = 0;  // down's folded-combine arrival counters, one per 32 rows of H
    int xflags = 0, hflags = 0;
    int64_t ntiles = 0;
};

// Slots in first-appearance order over (row, choice) -- the order in which
// moe_forward groups rows by expert (model.rs:219-233).  Invalid ids (out of
// range or not loaded) set the sticky error flag and contribute nothing.
// Whole-workgroup function: ids are read once in parallel, the assignment
// runs in LDS, the plan is written out in parallel.  n = M*k <= 256.
// tbl: the [6][E] pointer table (ExpertPtrs laid out from gate_w).
// The slot plan of make_plan for one activation row (n = k <= 64 entries),
// resolved by each wave on its own (lane j holds entry j; no LDS, no
// barrier): returns the slot count and lane `slot u's first entry`'s
// pointers in p6 (unset when u >= count).  The writer wave also writes the
// plan and the invalid-id flag exactly as make_plan does.  id: this lane's
// entry (-1 past n), loaded by the caller ahead of other loads.
__device__ inline int plan_slot_wave(int id, int n, int64_t E, const void *const *__restrict__ tbl,
                                     int u, bool writer, MoePlan plan,
                                     int32_t *__restrict__ err_flag, const void *(&p6)[6]) {
    const int lane = threadIdx.x & 63;
    const bool inr = lane < n && id >= 0 && id < E;
    const int64_t ec = inr ? id : 0;
    const void *p[6];
#pragma unroll
    for (int i = 0; i < 6; i++) p[i] = tbl[(int64_t)i * E + ec];
    const bool ok = inr && p[kSpGate] != nullptr;
    const int e = ok ? id : -1;
    // j0: the entry's first appearance (the reference groups rows by expert
    // in first-appearance order, model.rs:219-233)
    int j0 = lane;
    for (int i = 0; i < n; i++) {
        const int ei = __builtin_amdgcn_readlane(e, i);
        if (i < j0 && ei == e) j0 = i;
    }
    const bool first = ok && j0 == lane;
    const uint64_t fm = __ballot(first);
    const int slot = ok ? __popcll(fm & ((1ull << j0) - 1)) : -1;
    const int cnt = __popcll(fm);
    const uint64_t um = __ballot(first && slot == u);
    if (um) {
        const int L = __ffsll((unsigned long long)um) - 1;
#pragma unroll
        for (int i = 0; i < 6; i++) {
            const uint64_t v = (uint64_t)p[i];
            const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, L);
            const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), L);
            p6[i] = (const void *)(((uint64_t)hi << 32) | lo);
        }
    }
    if (writer) {
        if (lane < n) {
            if (!ok && id != -1 && err_flag) *err_flag = 1;
            plan.choice_slot[lane] = slot;
            if (first) {
                plan.uniq[slot] = e;
#pragma unroll
                for (int i = 0; i < 6; i++) plan.sp[slot * 6 + i] = p[i];
            }
        }
        if (lane == 0) *plan.count = cnt;
    }
    return cnt;
}

__device__ inline void make_plan(const int32_t *ids, int M, int k, int E,
                          const void *const *__restrict__ tbl, int extra_slot,
                          MoePlan plan, int32_t *__restrict__ err_flag) {
    if (M * k <= 64 && extra_slot < 0) {
        // up to 64 entries: wave 0 alone, one entry per lane (the same plan)
        if ((threadIdx.x >> 6) == 0) {
            const int lane = threadIdx.x & 63;
            const void *p6[6];
            plan_slot_wave(lane < M * k ? ids[lane] : -1, M * k, E, tbl, 0, true, plan, err_flag, p6);
        }
        return;
    }
    const void *const *gate_tbl = tbl;
    __shared__ int s_e[256], s_first[256];
    const int n = M * k, tid = threadIdx.x;
    if (tid < n) {
        const int e = ids[tid];
        const bool ok = e >= 0 && e < E && gate_tbl[e] != nullptr;
        if (!ok && e != -1 && err_flag) *err_flag = 1;
        s_e[tid] = ok ? e : -1;
    }
    __syncthreads();
    // entry i opens a slot when its expert does not appear before it
    int e = -1, j0 = -1;
    if (tid < n) {
        e = s_e[tid];
        if (e >= 0) {
            j0 = tid;
            for (int j = 0; j < tid; j++)
                if (s_e[j] == e) { j0 = j; break; }
        }
        s_first[tid] = e >= 0 && j0 == tid;
    }
    __syncthreads();
    if (tid < n) {
        // slot = number of slot openings before the expert's first entry
        int slot = -1;
        if (e >= 0) {
            slot = 0;
            for (int j = 0; j < j0; j++) slot += s_first[j];
            if (j0 == tid) {
                plan.uniq[slot] = e;
#pragma unroll
                for (int i = 0; i < 6; i++) plan.sp[slot * 6 + i] = tbl[(int64_t)i * E + e];
            }
        }
        plan.choice_slot[tid] = slot;
    }
    if (tid == 0) {
        int U = 0;
        for (int j = 0; j < n; j++) U += s_first[j];
        if (extra_slot >= 0) {  // a dense MLP run as one more slot
            for (int i = 0; i < 6; i++) plan.sp[U * 6 + i] = tbl[(int64_t)i * E + extra_slot];
            plan.uniq[U++] = extra_slot;
        }
        *plan.count = U;
    }
}

inline int64_t moe_slots(int M, int64_t k, int64_t E, int extra) {
    int64_t s = (int64_t)M * k;
    if (s > E) s = E;
    return s + (extra >= 0 ? 1 : 0);
}
ScratchLayout moe_layout(int64_t M, int64_t k, int64_t slots, int64_t H, int64_t I, int fmt);
size_t moe_scratch_bytes(int64_t M, int64_t k, int64_t slots, int64_t H, int64_t I, int fmt);
bool moe_shape_ok(int fmt, int64_t H, int64_t I);
// Whether routed experts of format fa and a shared MLP of format fb can run
// in the same launches.
inline bool moe_dual_ok(int fa, int fb) {
    return (fa == UT_FMT_INT4 || fa == UT_FMT_INT8) && (fb == UT_FMT_INT4 || fb == UT_FMT_INT8);
}
// scratch: device memory of moe_layout(...).total bytes for this call's
// (M, k, slots); slots from moe_slots().
int32_t moe_pass(ut_ctx *ctx, const MoeCall &c, void *scratch);
// The plan buffers inside a pass's scratch.
MoePlan moe_plan_view(void *scratch, const ScratchLayout &L);
// Routes M <= 4 rows and writes the slot plan into `plan` in one launch.
// parts (optional): the gate GEMV's deferred split-K partials, summed here
// instead of logits being read.
int32_t launch_route_plan(ut_ctx *ctx, const float *logits, const SplitKPartials *parts,
                          const float *bias, int M, int64_t E, int32_t k, int32_t n_group,
                          int32_t topk_group, int32_t norm, float scale, int32_t *ids,
                          float *weights, const void *const *tbl, MoePlan plan,
                          int32_t *err_flag);

int32_t launch_route(ut_ctx *ctx, const float *logits, const float *bias, int64_t rows,
                     int64_t E, int32_t k, int32_t n_group, int32_t topk_group, int32_t norm,
                     float scale, int32_t *ids, float *weights);

// Digitise rows of x in slot groups of rows_per_slot rows; groups at or past
// *slot_count are skipped.
// Digitise x [M, K] and, in one extra workgroup of the same launch, build
// the slot plan of (ids, M, k) -- the two independent set-up steps of an
// expert pass.
int32_t launch_digitize_plan(ut_ctx *ctx, const float *x, int64_t M, int64_t K, XDigits xd,
                             int flags, const int32_t *ids, int k, int64_t E,
                             const void *const *tbl, MoePlan plan, int32_t *err_flag);

int32_t launch_digitize_slots(ut_ctx *ctx, const float *x, int64_t ldx, int64_t M, int64_t K,
                              const uint32_t *rowmax_parts, int32_t nparts, XDigits xd,
                              int flags, const int32_t *slot_count, int rows_per_slot);

}  // namespace ut
