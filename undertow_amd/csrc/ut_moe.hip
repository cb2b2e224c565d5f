// ut_moe.hip -- the routed-expert block of moe_forward on gfx950
// (adapters/undertow-deepseek-moe/src/model.rs:195-286) and the DeepSeek
// sigmoid router (router.rs:58-113, undertow-core/src/router.rs:136-163).
//
// One pass over M <= 4 token rows:
//   k_route_wave   one wavefront per row: sigmoid, bias, group limitation,
//                  top-k by rank (value desc, lowest index first), weights
//                  (k_route: the workgroup form for other expert counts)
//   slot plan      unique experts in first-appearance order -> slots; built
//                  by every gate/up wave itself when M*k <= 64 (else by
//                  k_moe_plan, k_route_plan_wave or the digitiser)
//   k_moe_gate_up  grid (I/16, slots): gate and up rows of one expert in the
//                  same lanes, h = silu(g)*u written per (slot, row), plus
//                  per-workgroup max|h| partials; at one row it may also
//                  route the row and digitise x while staging it
//   k_moe_down     grid (H/32, slots): d = down(h) per (slot, row),
//                  h digitised while it is staged (exponent from the partials)
//   k_moe_gate_up_mfma / k_moe_down_mfma  the same two stages on the
//                  matrix cores for int4 experts at 2..4 rows (ut_gemv_mfma.h),
//                  bit-identical results
//   k_moe_combine4 out[s] = sum_c w[s,c]*d[slot(s,c), s] in router order
//                  (k_moe_combine_norm: also the next rmsnorm + digits)
// Every expert's weights are read once per pass whatever rows chose it;
// the row dimension rides along in the same instructions.
#include <mutex>
#include "ut_gemv_core.h"
#include "ut_moe.h"
#include "ut_gemv_mfma.h"
#include "ut_rowdig.h"
#include "ut_ops.h"


namespace ut {

// ------------------------------------------------------------- router ---
__device__ __forceinline__ bool ranks_before(float a, int ia, float b, int ib) {
    // `a` precedes `b` in topk_indices order: larger value, or equal value
    // and lower index.
    return a > b || (a == b && ia < ib);
}

// Routes one row with the whole workgroup.  sm: 2*E + n_group floats.
__device__ __forceinline__ void route_row(const float *__restrict__ lg,
                                          const float *__restrict__ bias, int E, int k,
                                          int n_group, int topk_group, int norm, float scale,
                                          int32_t *__restrict__ ids, float *__restrict__ weights,
                                          float *sm, int *s_ids, int *s_group_ok) {
    __shared__ float s_w[64];  // sigmoid of the chosen, in choice order
    float *sc = sm;           // sigmoid scores
    float *corr = sm + E;     // corrected (selection) scores, then masked
    float *gsc = sm + 2 * E;  // group scores
    const int tid = threadIdx.x;
    if (tid < 64) s_ids[tid] = 0;
    for (int e = tid; e < E; e += blockDim.x) {
        float s = 1.0f / (1.0f + expf(-lg[e]));  // sigmoid (undertow-quant/src/lib.rs:116)
        sc[e] = s;
        corr[e] = bias ? __fadd_rn(s, bias[e]) : s;
    }
    __syncthreads();
    const bool limit = n_group > 1 && topk_group < n_group;
    if (limit) {
        const int gs = E / n_group;
        // group score = sum of the group's top-2 (in topk order: best first)
        for (int g = tid; g < n_group; g += blockDim.x) {
            const float *v = corr + g * gs;
            int b0 = 0;
            float v0 = v[0];
#pragma unroll 8
            for (int i = 1; i < gs; i++) {
                const float vi = v[i];
                if (vi > v0) { b0 = i; v0 = vi; }
            }
            float s = 0.0f + v0;
            if (gs > 1) {
                int b1 = b0 == 0 ? 1 : 0;
                float v1 = v[b1];
#pragma unroll 8
                for (int i = 0; i < gs; i++) {
                    const float vi = v[i];
                    if (i != b0 && ranks_before(vi, i, v1, b1)) { b1 = i; v1 = vi; }
                }
                s = s + v1;
            }
            gsc[g] = s;
        }
        __syncthreads();
        for (int g = tid; g < n_group; g += blockDim.x) {
            int rank = 0;
            for (int j = 0; j < n_group; j++) rank += ranks_before(gsc[j], j, gsc[g], g);
            s_group_ok[g] = rank < topk_group;
        }
        __syncthreads();
        for (int e = tid; e < E; e += blockDim.x) {
            int g = e / gs;
            bool ok = g < n_group && s_group_ok[g];
            if (!ok) corr[e] = -INFINITY;
        }
        __syncthreads();
    }
    const int keff = k < E ? k : E;
    for (int e = tid; e < E; e += blockDim.x) {
        const float v = corr[e];
        int rank = 0;
#pragma unroll 16
        for (int j = 0; j < E; j++) rank += ranks_before(corr[j], j, v, e);
        if (rank < keff) {
            s_ids[rank] = e;
            s_w[rank] = sc[e];
        }
    }
    __syncthreads();
    // weights = sigmoid of the chosen, normalised by their sequential sum
    // (+1e-20) in choice order, then scaled
    if (tid < k) {
        if (tid < keff) {
            float denom = 0.0f;
            for (int j = 0; j < keff; j++) denom = denom + s_w[j];
            denom = denom + 1e-20f;
            const float w = s_w[tid];
            const float v = norm ? w / denom : w;
            ids[tid] = s_ids[tid];
            weights[tid] = __fmul_rn(v, scale);
        } else {  // k > E: no expert (contributes nothing)
            ids[tid] = -1;
            weights[tid] = 0.0f;
        }
    }
    __syncthreads();
}

// ------------------------------------------------------ wave router ---
// The same routing by one wavefront: lane l holds experts
// [l*KPL, l*KPL + KPL), and every selection is a cross-lane max of 64-bit
// keys = order-preserving value bits above the complemented expert index,
// so the largest key is the largest value with the lowest index (the
// order of topk_indices, undertow-core/src/router.rs:136-163).  The group
// scores come from max reductions over each group's run of lanes.  -0 is
// keyed as +0 (the two compare equal in the reference).  Taken when
// E <= 64*KPL and, with group limitation, E = n_group * gs with gs a
// power-of-two multiple of KPL (gs/KPL <= 64 lanes per group).

__device__ __forceinline__ uint32_t order_bits(float v) {
    const uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float order_value(uint32_t h) {
    return __uint_as_float((h & 0x80000000u) ? (h & 0x7fffffffu) : ~h);
}
__device__ __forceinline__ uint64_t route_key(float v, int e) {
    return ((uint64_t)order_bits(v) << 32) | (uint64_t)(uint32_t)~(uint32_t)e;
}

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xF, false);
}
// max over aligned runs of LG lanes, valid in the run's last lane (and in
// every lane of the run for LG <= 16)
template <int LG>
__device__ __forceinline__ uint32_t run_max_u32(uint32_t v) {
    if constexpr (LG >= 2) v = max(v, dpp_u32<0xB1>(v));        // quad_perm 1,0,3,2
    if constexpr (LG >= 4) v = max(v, dpp_u32<0x4E>(v));        // quad_perm 2,3,0,1
    if constexpr (LG >= 8) v = max(v, dpp_u32<0x141>(v));       // row_half_mirror
    if constexpr (LG >= 16) v = max(v, dpp_u32<0x140>(v));      // row_mirror
    if constexpr (LG >= 32) v = max(v, dpp_u32<0x142, 0xA>(v)); // row_bcast15
    if constexpr (LG >= 64) v = max(v, dpp_u32<0x143, 0xC>(v)); // row_bcast31
    return v;
}
// the run's maximum key in every lane of the run
template <int LG>
__device__ __forceinline__ uint64_t run_max_key(uint64_t k) {
    const int lane = threadIdx.x & 63, last = lane | (LG - 1);
    uint32_t hi = run_max_u32<LG>((uint32_t)(k >> 32));
    if constexpr (LG == 64) hi = __builtin_amdgcn_readlane(hi, 63);
    else if constexpr (LG == 32) hi = __shfl(hi, last, 64);
    uint32_t lo = run_max_u32<LG>((uint32_t)(k >> 32) == hi ? (uint32_t)k : 0u);
    if constexpr (LG == 64) lo = __builtin_amdgcn_readlane(lo, 63);
    else if constexpr (LG == 32) lo = __shfl(lo, last, 64);
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t run_max_key_rt(uint64_t k, int LG) {
    switch (LG) {
    case 1: return k;
    case 2: return run_max_key<2>(k);
    case 4: return run_max_key<4>(k);
    case 8: return run_max_key<8>(k);
    case 16: return run_max_key<16>(k);
    case 32: return run_max_key<32>(k);
    default: return run_max_key<64>(k);
    }
}

static bool route_wave_ok(int64_t E, int n_group, int topk_group, int k, int *kpl) {
    int p = E <= 64 ? 1 : E <= 128 ? 2 : E <= 256 ? 4 : E <= 512 ? 8 : E <= 1024 ? 16 : 0;
    if (!p || k > 64) return false;
    *kpl = p;
    if (!(n_group > 1 && topk_group < n_group)) return true;
    if (E % n_group) return false;
    const int64_t gs = E / n_group, lg = gs / p;
    return gs % p == 0 && lg >= 1 && lg <= 64 && (lg & (lg - 1)) == 0;
}

// Routes one row with one wavefront (all 64 lanes active).  Lane r < k
// returns choice r in *my_id / *my_w (id -1, weight 0 past E).
// This lane's logits and biases (experts lane*KPL + j), loaded ahead of the
// routing so a caller can overlap the loads with other work.
template <int KPL>
__device__ __forceinline__ void route_load(const float *__restrict__ lg,
                                           const float *__restrict__ bias, int E,
                                           float (&lv)[KPL], float (&bv)[KPL]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < KPL; j++) {
        const int e = lane * KPL + j;
        lv[j] = e < E ? lg[e] : 0.0f;
        bv[j] = e < E && bias ? bias[e] : 0.0f;
    }
}

template <int KPL>
__device__ __forceinline__ void route_row_wave_v(const float (&lv)[KPL], const float (&bv)[KPL],
                                                 bool has_bias, int E, int k, int n_group,
                                                 int topk_group, int norm, float scale,
                                                 int32_t *my_id, float *my_w);

template <int KPL>
__device__ __forceinline__ void route_row_wave(const float *__restrict__ lg,
                                               const float *__restrict__ bias, int E, int k,
                                               int n_group, int topk_group, int norm, float scale,
                                               int32_t *my_id, float *my_w) {
    float lv[KPL], bv[KPL];
    route_load<KPL>(lg, bias, E, lv, bv);
    route_row_wave_v<KPL>(lv, bv, bias != nullptr, E, k, n_group, topk_group, norm, scale, my_id,
                          my_w);
}

// The wave router on loaded logits (route_load), in three phases for
// callers that interleave them with other work: the keys (sigmoid, bias),
// the group limitation, and the selections with their weights.
template <int KPL>
__device__ __forceinline__ void route_phase_keys(const float (&lv)[KPL], const float (&bv)[KPL],
                                                 bool has_bias, int E, float (&sc)[KPL],
                                                 uint64_t (&key)[KPL]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < KPL; j++) {
        const int e = lane * KPL + j;
        if (e < E) {
            const float s = 1.0f / (1.0f + expf(-lv[j]));  // sigmoid (undertow-quant/src/lib.rs:116)
            sc[j] = s;
            key[j] = route_key(has_bias ? __fadd_rn(s, bv[j]) : s, e);
        } else {
            sc[j] = 0.0f;
            key[j] = 0;  // below every expert's key
        }
    }
}

// CLG > 0: the group's lane run known at compile time (CLG lanes, which the
// caller checked); the same steps without the run-length switch.
template <int KPL, int CLG = 0>
__device__ __forceinline__ void route_phase_groups(uint64_t (&key)[KPL], int E, int n_group,
                                                   int topk_group) {
    const int lane = threadIdx.x & 63;
    if (n_group > 1 && topk_group < n_group) {
        const int gs = E / n_group, LG = CLG > 0 ? CLG : gs / KPL;
        uint64_t b = key[0];
#pragma unroll
        for (int j = 1; j < KPL; j++) b = key[j] > b ? key[j] : b;
        uint64_t m1;
        if constexpr (CLG > 0) m1 = run_max_key<CLG>(b);
        else m1 = run_max_key_rt(b, LG);
        uint64_t b2 = 0;
#pragma unroll
        for (int j = 0; j < KPL; j++) b2 = key[j] != m1 && key[j] > b2 ? key[j] : b2;
        uint64_t m2;
        if constexpr (CLG > 0) m2 = run_max_key<CLG>(b2);
        else m2 = run_max_key_rt(b2, LG);
        // group score = sum of the group's top-2 in topk order
        float gsum = 0.0f + order_value((uint32_t)(m1 >> 32));
        if (gs > 1) gsum = gsum + order_value((uint32_t)(m2 >> 32));
        const int g = lane / LG;
        const uint64_t gk = route_key(gsum, g);
        // group g2's key from its first lane (a wave-uniform lane: read
        // lanes, no LDS permutes)
        int rank = 0;
        if constexpr (CLG > 0) {
#pragma unroll
            for (int g2 = 0; g2 < 64 / CLG; g2++) {
                const uint32_t ohi = __builtin_amdgcn_readlane((uint32_t)(gk >> 32), g2 * CLG);
                const uint32_t olo = __builtin_amdgcn_readlane((uint32_t)gk, g2 * CLG);
                rank += g2 < n_group && (((uint64_t)ohi << 32) | olo) > gk;
            }
        } else {
            for (int g2 = 0; g2 < n_group; g2++) {
                const int src = g2 * LG;
                const uint32_t ohi = __builtin_amdgcn_readlane((uint32_t)(gk >> 32), src);
                const uint32_t olo = __builtin_amdgcn_readlane((uint32_t)gk, src);
                rank += (((uint64_t)ohi << 32) | olo) > gk;
            }
        }
        if (rank >= topk_group) {
#pragma unroll
            for (int j = 0; j < KPL; j++)
                if (lane * KPL + j < E) key[j] = route_key(-INFINITY, lane * KPL + j);
        }
    }
}

template <int KPL>
__device__ __forceinline__ void route_phase_select(const float (&sc)[KPL],
                                                   const uint64_t (&key)[KPL], int E, int k,
                                                   int norm, float scale, int32_t *my_id,
                                                   float *my_w) {
    const int lane = threadIdx.x & 63;
    // the selections: the largest value bits over the wave, then the lowest
    // index holding them -- the lowest lane with a match, its lowest j
    // (e = lane*KPL + j) -- which is the largest 64-bit key without a second
    // reduction.  A chosen key drops to 0, below every expert's value bits
    // (-inf keys as 0x007fffff); only keys past E are 0, and at most E are
    // chosen.
    uint32_t hk[KPL];
#pragma unroll
    for (int j = 0; j < KPL; j++) hk[j] = (uint32_t)(key[j] >> 32);
    const int keff = k < E ? k : E;
    float denom = 0.0f;
    int32_t id = -1;
    float wv = 0.0f;
    for (int r = 0; r < keff; r++) {
        uint32_t b = hk[0];
#pragma unroll
        for (int j = 1; j < KPL; j++) b = max(b, hk[j]);
        const uint32_t mx = __builtin_amdgcn_readlane(run_max_u32<64>(b), 63);
        int jf = -1;
        float sj = 0.0f;
#pragma unroll
        for (int j = KPL - 1; j >= 0; j--)
            if (hk[j] == mx) {
                jf = j;
                sj = sc[j];
            }
        const int L = __ffsll((unsigned long long)__ballot(jf >= 0)) - 1;
        const int jw = __builtin_amdgcn_readlane(jf, L);
        const int e = L * KPL + jw;
        const float sv = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(sj), L));
        if (lane == L)
#pragma unroll
            for (int j = 0; j < KPL; j++)
                if (j == jw) hk[j] = 0;
        denom = denom + sv;  // sequential sum in choice order
        if (lane == r) { id = e; wv = sv; }
    }
    // weights = sigmoid of the chosen, normalised by their sum (+1e-20)
    denom = denom + 1e-20f;
    if (lane < k) {
        if (lane < keff) {
            *my_id = id;
            *my_w = __fmul_rn(norm ? wv / denom : wv, scale);
        } else {  // k > E: no expert (contributes nothing)
            *my_id = -1;
            *my_w = 0.0f;
        }
    }
}

template <int KPL>
__device__ __forceinline__ void route_row_wave_v(const float (&lv)[KPL], const float (&bv)[KPL],
                                                 bool has_bias, int E, int k, int n_group,
                                                 int topk_group, int norm, float scale,
                                                 int32_t *my_id, float *my_w) {
    float sc[KPL];
    uint64_t key[KPL];
    route_phase_keys<KPL>(lv, bv, has_bias, E, sc, key);
    route_phase_groups<KPL>(key, E, n_group, topk_group);
    route_phase_select<KPL>(sc, key, E, k, norm, scale, my_id, my_w);
}

template <int KPL>
__global__ __launch_bounds__(64) void k_route_wave(const float *__restrict__ logits,
                                                   const float *__restrict__ bias, int E, int k,
                                                   int n_group, int topk_group, int norm,
                                                   float scale, int32_t *__restrict__ ids,
                                                   float *__restrict__ weights) {
    const int row = blockIdx.x, lane = threadIdx.x;
    int32_t id = -1;
    float w = 0.0f;
    route_row_wave<KPL>(logits + (int64_t)row * E, bias, E, k, n_group, topk_group, norm, scale,
                        &id, &w);
    if (lane < k) {
        ids[(int64_t)row * k + lane] = id;
        weights[(int64_t)row * k + lane] = w;
    }
}

__global__ __launch_bounds__(256) void k_route(const float *__restrict__ logits,
                                               const float *__restrict__ bias, int E, int k,
                                               int n_group, int topk_group, int norm,
                                               float scale, int32_t *__restrict__ ids,
                                               float *__restrict__ weights) {
    extern __shared__ float sm[];
    __shared__ int s_ids[64];
    __shared__ int s_group_ok[64];
    const int row = blockIdx.x;
    route_row(logits + (int64_t)row * E, bias, E, k, n_group, topk_group, norm, scale,
              ids + (int64_t)row * k, weights + (int64_t)row * k, sm, s_ids, s_group_ok);
}

// Routing of M <= 4 rows plus the slot plan in one workgroup (one launch on
// the decode path instead of two).
// logits: [M, E], or (part != nullptr) the gate GEMV's split-K partials
// [ks][M][E] (f32 bits), summed here in z order as the GEMV's own sum
// launch would.
__global__ __launch_bounds__(256) void k_route_plan(const float *__restrict__ logits,
                                                    const int64_t *__restrict__ part, int ks,
                                                    const float *__restrict__ bias, int M, int E,
                                                    int k, int n_group, int topk_group, int norm,
                                                    float scale, int32_t *__restrict__ ids,
                                                    float *__restrict__ weights,
                                                    const void *const *__restrict__ tbl,
                                                    MoePlan plan, int32_t *__restrict__ err_flag) {
    extern __shared__ float sm[];  // [2E + n_group] route scratch, then [M][E] logits
    __shared__ int s_ids[64];
    __shared__ int s_group_ok[64];
    __shared__ int32_t s_all[4 * 64];
    float *s_lg = sm + 2 * E + (n_group > 0 ? n_group : 1);
    for (int i = threadIdx.x; i < M * E; i += blockDim.x) {
        float v;
        if (part) {
            v = __uint_as_float((uint32_t)part[i]);
#pragma unroll 16
            for (int z = 1; z < ks; z++) v = __fadd_rn(v, __uint_as_float((uint32_t)part[(int64_t)z * M * E + i]));
        } else {
            v = logits[i];
        }
        s_lg[i] = v;
    }
    __syncthreads();
    for (int row = 0; row < M; row++) {
        route_row(s_lg + row * E, bias, E, k, n_group, topk_group, norm, scale,
                  ids + (int64_t)row * k, weights + (int64_t)row * k, sm, s_ids, s_group_ok);
        // the chosen ids from LDS (route_row ends with a barrier)
        if (threadIdx.x < k) s_all[row * k + threadIdx.x] = threadIdx.x < (k < E ? k : E) ? s_ids[threadIdx.x] : -1;
        __syncthreads();
    }
    __syncthreads();
    make_plan(s_all, M, k, E, tbl, -1, plan, err_flag);
}

// k_route_plan with the wave router: wave r routes row r (M <= 4).
template <int KPL>
__global__ __launch_bounds__(256) void k_route_plan_wave(const float *__restrict__ logits,
                                                         const int64_t *__restrict__ part, int ks,
                                                         const float *__restrict__ bias, int M,
                                                         int E, int k, int n_group, int topk_group,
                                                         int norm, float scale,
                                                         int32_t *__restrict__ ids,
                                                         float *__restrict__ weights,
                                                         const void *const *__restrict__ tbl,
                                                         MoePlan plan, int32_t *__restrict__ err_flag) {
    extern __shared__ float s_lg[];  // [M][E] logits
    __shared__ int32_t s_all[4 * 64];
    for (int i = threadIdx.x; i < M * E; i += blockDim.x) {
        float v;
        if (part) {
            v = __uint_as_float((uint32_t)part[i]);
#pragma unroll 16
            for (int z = 1; z < ks; z++) v = __fadd_rn(v, __uint_as_float((uint32_t)part[(int64_t)z * M * E + i]));
        } else {
            v = logits[i];
        }
        s_lg[i] = v;
    }
    __syncthreads();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (wave < M) {
        int32_t id = -1;
        float w = 0.0f;
        route_row_wave<KPL>(s_lg + wave * E, bias, E, k, n_group, topk_group, norm, scale, &id, &w);
        if (lane < k) {
            ids[(int64_t)wave * k + lane] = id;
            weights[(int64_t)wave * k + lane] = w;
            s_all[wave * k + lane] = id;
        }
    }
    __syncthreads();
    make_plan(s_all, M, k, E, tbl, -1, plan, err_flag);
}

__global__ __launch_bounds__(256) void k_moe_plan(const int32_t *__restrict__ ids, int M, int k, int E,
                           const void *const *__restrict__ tbl, int extra_slot,
                           MoePlan plan, int32_t *__restrict__ err_flag) {
    make_plan(ids, M, k, E, tbl, extra_slot, plan, err_flag);
}

int32_t launch_route(ut_ctx *ctx, const float *logits, const float *bias, int64_t rows,
                     int64_t E, int32_t k, int32_t n_group, int32_t topk_group, int32_t norm,
                     float scale, int32_t *ids, float *weights) {
    if (rows <= 0) return UT_OK;
    size_t shmem = (size_t)(2 * E + (n_group > 0 ? n_group : 1)) * sizeof(float);
    int tok = timing_begin(ctx, "route");
    int kpl = 0;
    if (route_wave_ok(E, n_group, topk_group, k, &kpl)) {
#define UT_ROUTE_W(P)                                                                          \
    hipLaunchKernelGGL(k_route_wave<P>, dim3((unsigned)rows), dim3(64), 0, ctx->stream, logits, \
                       bias, (int)E, (int)k, (int)n_group, (int)topk_group, (int)norm, scale, ids, \
                       weights)
        switch (kpl) {
        case 1: UT_ROUTE_W(1); break;
        case 2: UT_ROUTE_W(2); break;
        case 4: UT_ROUTE_W(4); break;
        case 8: UT_ROUTE_W(8); break;
        default: UT_ROUTE_W(16); break;
        }
#undef UT_ROUTE_W
    } else {
        hipLaunchKernelGGL(k_route, dim3((unsigned)rows), dim3(256), shmem, ctx->stream, logits, bias,
                           (int)E, (int)k, (int)n_group, (int)topk_group, (int)norm, scale, ids,
                           weights);
    }
    timing_end(ctx, tok);
    return launch_check(ctx, "k_route");
}

int32_t launch_route_plan(ut_ctx *ctx, const float *logits, const SplitKPartials *parts,
                          const float *bias, int M, int64_t E, int32_t k, int32_t n_group,
                          int32_t topk_group, int32_t norm, float scale, int32_t *ids,
                          float *weights, const void *const *tbl, MoePlan plan,
                          int32_t *err_flag) {
    if (M < 1 || M > 4 || k > 64) {
        set_error(ctx, "route_plan: M=%d k=%d outside 1..4 / 1..64", M, k);
        return UT_ERR_ARG;
    }
    const bool split = parts && parts->ks > 1;
    if (split && parts->O != E) {
        set_error(ctx, "route_plan: partials of %lld rows for %lld experts", (long long)parts->O,
                  (long long)E);
        return UT_ERR_ARG;
    }
    size_t shmem = (size_t)(2 * E + (n_group > 0 ? n_group : 1) + M * E) * sizeof(float);
    int tok = timing_begin(ctx, "route_plan");
    int kpl = 0;
    if (route_wave_ok(E, n_group, topk_group, k, &kpl)) {
#define UT_ROUTE_PW(P)                                                                           \
    hipLaunchKernelGGL(k_route_plan_wave<P>, dim3(1), dim3(256), (size_t)M * E * sizeof(float),   \
                       ctx->stream, logits, split ? (const int64_t *)parts->part : nullptr,      \
                       split ? parts->ks : 1, bias, M, (int)E, (int)k, (int)n_group,              \
                       (int)topk_group, (int)norm, scale, ids, weights, tbl, plan, err_flag)
        switch (kpl) {
        case 1: UT_ROUTE_PW(1); break;
        case 2: UT_ROUTE_PW(2); break;
        case 4: UT_ROUTE_PW(4); break;
        case 8: UT_ROUTE_PW(8); break;
        default: UT_ROUTE_PW(16); break;
        }
#undef UT_ROUTE_PW
    } else {
        hipLaunchKernelGGL(k_route_plan, dim3(1), dim3(256), shmem, ctx->stream, logits,
                           split ? (const int64_t *)parts->part : nullptr, split ? parts->ks : 1, bias, M,
                           (int)E, (int)k, (int)n_group, (int)topk_group, (int)norm, scale, ids,
                           weights, tbl, plan, err_flag);
    }
    timing_end(ctx, tok);
    return launch_check(ctx, "k_route_plan");
}

// --------------------------------------------------------- gate / up ---
struct GateUpArgs {
    ExpertPtrs tbl;
    const void *const *sp;  // the plan's per-slot weight pointers
    const int32_t *uniq;
    const int32_t *count;
    int64_t H, I, row_bytes;  // gate/up are [I, H]
    XSrc x;                   // digits (or f32) of x, shared by all slots
    const int32_t *exps;
    const float *mfma_xf = nullptr;  // k_moe_gate_up_mfma: x as f32 [M][H] (digitised by exps)
    bool mfma8 = false;              // k_moe_gate_up_i8_mfma: int8 experts, x as digit planes
    float *h;                 // [slots][M][I]
    uint32_t *hmax_parts;     // [slots][M][ntiles] float bits
    int ntiles;
    // optional (plan_ids set; M * k <= 64): every wave resolves its slot
    // from the expert ids itself and workgroup (0, 0) writes the plan for
    // the later launches, so no plan launch runs first
    const int32_t *plan_ids = nullptr;
    int plan_M = 0, plan_k = 0;
    int64_t E = 0;
    const void *const *ptbl = nullptr;  // [6][E] pointer table
    MoePlan plan{};
    int32_t *err_flag = nullptr;
    // optional (one row, with plan_ids' conditions, E/64 = 4 keys per
    // lane): the waves route the row from the logits first; workgroup
    // (0, 0) writes the choices to route_ids / route_w
    const float *route_lg = nullptr;
    const float *route_bias = nullptr;
    int route_ng = 1, route_tg = 1, route_norm = 0;
    float route_scale = 1.0f;
    int32_t *route_ids = nullptr;
    float *route_w = nullptr;
    // optional: zeroed by workgroup (0, 0) for the down launch that follows
    // (its folded combine's arrival counters, CombineFold)
    int32_t *arrive = nullptr;
    int narrive = 0;
};

// UT_MOE_FOLD_COMBINE=1: fold the routed combine into down (CombineFold)
// instead of a combine launch after it.
#ifndef UT_MOE_FOLD_COMBINE
#define UT_MOE_FOLD_COMBINE 0
#endif
// (the fold's device code is compiled in only with the switch on: its
// argument loads and branches cost the default kernels registers)

// Workgroup (0, 0) of a gate/up launch clears the next down launch's
// arrival counters (stream order makes them zero when down starts).
__device__ __forceinline__ void clear_arrivals(const GateUpArgs &a, int u, int tile) {
    if constexpr (UT_MOE_FOLD_COMBINE) {
        if (a.arrive && u == 0 && tile == 0)
            for (int i = threadIdx.x; i < a.narrive; i += blockDim.x) a.arrive[i] = 0;
    }
}

// plan_slot_wave for choices made in this launch whose gate and up weight
// pointers came with them (gsel, usel: lane j < n holds entry j's), so the
// slot's weights can be read at once; slot u's scale pointers are loaded by
// expert id afterwards (read only after the weights).  The writer wave loads
// all six pointers per entry for the plan, as plan_slot_wave.
__device__ inline int plan_slot_wave_pf(int id, int n, int64_t E,
                                        const void *const *__restrict__ tbl, uint64_t gsel,
                                        uint64_t usel, int u, bool writer, MoePlan plan,
                                        int32_t *__restrict__ err_flag, const void *(&p6)[6]) {
    const int lane = threadIdx.x & 63;
    const bool inr = lane < n && id >= 0 && id < E;
    const bool ok = inr && gsel != 0;
    const int e = ok ? id : -1;
    // j0: the entry's first appearance (model.rs:219-233)
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
        // halves as uint32_t: readlane returns int, which would sign-extend
        const uint32_t glo = __builtin_amdgcn_readlane((uint32_t)gsel, L);
        const uint32_t ghi = __builtin_amdgcn_readlane((uint32_t)(gsel >> 32), L);
        const uint32_t ulo = __builtin_amdgcn_readlane((uint32_t)usel, L);
        const uint32_t uhi = __builtin_amdgcn_readlane((uint32_t)(usel >> 32), L);
        const int eu = __builtin_amdgcn_readlane(e, L);
        p6[kSpGate] = (const void *)(((uint64_t)ghi << 32) | glo);
        p6[kSpUp] = (const void *)(((uint64_t)uhi << 32) | ulo);
        p6[kSpGateS] = tbl[(int64_t)kSpGateS * E + eu];
        p6[kSpUpS] = tbl[(int64_t)kSpUpS * E + eu];
    }
    if (writer) {
        if (lane < n) {
            if (!ok && id != -1 && err_flag) *err_flag = 1;
            plan.choice_slot[lane] = slot;
            if (first) {
                plan.uniq[slot] = e;
#pragma unroll
                for (int i = 0; i < 6; i++) plan.sp[slot * 6 + i] = tbl[(int64_t)i * E + e];
            }
        }
        if (lane == 0) *plan.count = cnt;
    }
    return cnt;
}

// Gate/up at one row with the routing in this launch and x digitised here
// (f32 or bf16 activations, one staged chunk): wave 0 routes the row while
// waves 1-3 stage and digitise x, the router's phases falling between the
// staging's two workgroup barriers -- the keys before the one after the
// row-max partials, the group limitation and the selections before the
// one after the digits.  Wave 0 loads the logits and its experts' gate/up
// pointers first and hands the choices and their pointers over in LDS; the
// first weight loads follow at once.  The same digits, exponent, choices
// and results as the one-wave router in gemv_core's staging.  Returns the
// slot count; rows, scale pointers, exponent and res are set for slot u.
template <int FMT>
__device__ __forceinline__ int gate_up_route_staged(const GateUpArgs &a, int u, int tile,
                                                    int64_t oc, uint32_t *lds,
                                                    const uint8_t *(&rows)[2], const float *&gsc,
                                                    const float *&usc, int32_t &exl,
                                                    CoreOut<FMT, 1, 2> &res) {
    using T = FmtTraits<FMT>;
    constexpr int KC = gemv_chunk_cols<FMT, 1>();
    constexpr int CPW = T::kColsPerWord, PL = T::kPlanes, LW = KC / CPW, NV = CPW / 4;
    constexpr int NS = kGemvThreads - 64;  // staging threads (waves 1-3)
    constexpr int NI = (LW + NS - 1) / NS;
    __shared__ uint32_t s_red[4];
    __shared__ int32_t s_rid[64];
    __shared__ uint64_t s_gp[64], s_up[64];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, t = tid - 64;
    const int n = a.plan_k;  // one row
    const int E = (int)a.E;
    const int ng = (int)(a.H / CPW);  // word groups of the row
    const bool writer = u == 0 && tile == 0 && wave == 0;
    float lv[4], bv[4];
    uint64_t pg[4], pu[4];
    float4 v[NI][NV];
    if (wave == 0) {
        route_load<4>(a.route_lg, a.route_bias, E, lv, bv);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int e = lane * 4 + j;
            pg[j] = e < E ? (uint64_t)a.ptbl[(int64_t)kSpGate * E + e] : 0;
            pu[j] = e < E ? (uint64_t)a.ptbl[(int64_t)kSpUp * E + e] : 0;
        }
    } else {
#pragma unroll
        for (int j = 0; j < NI; j++) {
            const int i = t + j * NS, ic = i < ng ? i : ng - 1;
            if (a.x.xh) {
                const uint16_t *hs = a.x.xh + (int64_t)ic * CPW;
#pragma unroll
                for (int q = 0; q < NV; q++) {
                    // little-endian pairs: the low half is the even value
                    const uint2 hv = ld_global<uint2>(hs + 4 * q);
                    v[j][q] = make_float4(__uint_as_float(hv.x << 16),
                                          __uint_as_float(hv.x & 0xffff0000u),
                                          __uint_as_float(hv.y << 16),
                                          __uint_as_float(hv.y & 0xffff0000u));
                }
            } else {
#pragma unroll
                for (int q = 0; q < NV; q++)
                    v[j][q] = ld_global<float4>(a.x.xf + (int64_t)ic * CPW + 4 * q);
            }
        }
    }
    // phase 1: the keys | max|x| partials
    float rsc[4];
    uint64_t rkey[4];
    if (wave == 0) {
        __builtin_amdgcn_s_setprio(3);
        route_phase_keys<4>(lv, bv, a.route_bias != nullptr, E, rsc, rkey);
        if (lane == 0) s_red[0] = 0;
    } else {
        uint32_t b = 0;
#pragma unroll
        for (int j = 0; j < NI; j++)
            if (t + j * NS < ng)
#pragma unroll
                for (int q = 0; q < NV; q++)
                    b = max(b, max(max(__float_as_uint(fabsf(v[j][q].x)),
                                       __float_as_uint(fabsf(v[j][q].y))),
                                   max(__float_as_uint(fabsf(v[j][q].z)),
                                       __float_as_uint(fabsf(v[j][q].w)))));
        b = wave_reduce_dpp(b, [](uint32_t p, uint32_t q) { return p > q ? p : q; });
        if (lane == 0) s_red[wave] = b;
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    // the row's exponent, as rowmax_reduce
    const uint32_t r = max(max(s_red[0], s_red[1]), max(s_red[2], s_red[3]));
    int Ex = 0;
    if (r < 0x7f800000u && r != 0) (void)frexpf(__uint_as_float(r), &Ex);
    const int32_t sh = r >= 0x7f800000u ? INT32_MIN : 22 - Ex;
    exl = sh == INT32_MIN ? INT32_MIN : -sh;
    // phase 2: group limitation and selections | digits
    if (wave == 0) {
        // DeepSeek-V3's 8 groups of 32 experts: 8-lane runs at compile time
        if (a.route_ng > 0 && E == 32 * a.route_ng)
            route_phase_groups<4, 8>(rkey, E, a.route_ng, a.route_tg);
        else
            route_phase_groups<4>(rkey, E, a.route_ng, a.route_tg);
        int32_t rid = -1;
        float rw = 0.0f;
        route_phase_select<4>(rsc, rkey, E, a.plan_k, a.route_norm, a.route_scale, &rid, &rw);
        __builtin_amdgcn_s_setprio(0);
        // each choice's gate/up pointers from the lane holding its expert
        const bool inr = lane < n && rid >= 0 && rid < E;
        const int src = inr ? rid >> 2 : 0, jj = inr ? rid & 3 : 0;
        uint64_t gsel = 0, usel = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t glo = __shfl((uint32_t)pg[j], src, 64);
            const uint32_t ghi = __shfl((uint32_t)(pg[j] >> 32), src, 64);
            const uint32_t ulo = __shfl((uint32_t)pu[j], src, 64);
            const uint32_t uhi = __shfl((uint32_t)(pu[j] >> 32), src, 64);
            if (jj == j) {
                gsel = ((uint64_t)ghi << 32) | glo;
                usel = ((uint64_t)uhi << 32) | ulo;
            }
        }
        if (lane < n) {
            s_rid[lane] = rid;
            s_gp[lane] = gsel;
            s_up[lane] = usel;
        }
        if (writer && lane < n) {
            a.route_ids[lane] = rid;
            a.route_w[lane] = rw;
        }
    } else {
#pragma unroll
        for (int j = 0; j < NI; j++) {
            const int i = t + j * NS;
            if (i < ng) {
                float f[CPW];
#pragma unroll
                for (int q = 0; q < NV; q++) {
                    f[4 * q] = v[j][q].x; f[4 * q + 1] = v[j][q].y;
                    f[4 * q + 2] = v[j][q].z; f[4 * q + 3] = v[j][q].w;
                }
                uint32_t w[PL];
                digit_words<FMT>(f, CPW, sh, w);
#pragma unroll
                for (int p = 0; p < PL; p++) lds[p * LW + i] = w[p];
            }
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    const int id = lane < n ? s_rid[lane] : -1;
    const void *p6[6];
    const int cnt = plan_slot_wave_pf(id, n, a.E, a.ptbl, lane < n ? s_gp[lane] : 0,
                                      lane < n ? s_up[lane] : 0, u, writer, a.plan, a.err_flag,
                                      p6);
    const bool live = u < cnt;
    const uint8_t *dummy = a.x.xf ? (const uint8_t *)a.x.xf : (const uint8_t *)a.x.xh;
    rows[0] = live ? (const uint8_t *)p6[kSpGate] + oc * a.row_bytes : dummy;
    rows[1] = live ? (const uint8_t *)p6[kSpUp] + oc * a.row_bytes : dummy;
    gsc = live ? (const float *)p6[kSpGateS] : nullptr;
    usc = live ? (const float *)p6[kSpUpS] : nullptr;
    gemv_core<FMT, 1, 2, gemv_depth<1>(), KC, true>(rows, a.H, a.x, lds, res);
    return cnt;
}

// 16 h-rows per workgroup: wave w, row group g -> h row o = tile*16 +
// w*4 + g; row slot 0 reads gate row o, slot 1 up row o, so both land in the
// same lanes and h = silu(g)*u is formed in registers.
// STAGED_ROUTE: compile gate_up_route_staged in (launches whose one-row
// routing may come with x to digitise).
template <int FMT, int M, bool STAGED_ROUTE = true>
__device__ __forceinline__ void gate_up_body(const GateUpArgs &a, int u, int tile, uint32_t *lds,
                                             uint32_t *wg_max) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, s = lane & 15;
    const int64_t o = (int64_t)tile * kGateUpRowsPerWG + wave * 4 + g;
    const int64_t oc = o < a.I ? o : a.I - 1;
    const uint8_t *rows[2];
    const float *gsc = nullptr, *usc = nullptr;
    int cnt = 0;
    if (tid < 4) wg_max[tid] = 0;  // published by the core's barriers
    clear_arrivals(a, u, tile);
    CoreOut<FMT, M, 2> res;
    // x's exponents: given, or (self_max) found while x is staged (prep)
    int32_t exl[M];
    if constexpr (FMT != UT_FMT_F32)
        if (!a.x.self_max)
#pragma unroll
            for (int m = 0; m < M; m++) exl[m] = a.exps[m];
    auto prep = [&](int32_t (&shl)[4]) {
#pragma unroll
        for (int m = 0; m < M; m++) exl[m] = shl[m] == INT32_MIN ? INT32_MIN : -shl[m];
    };
    bool staged_route = false;
    if constexpr (STAGED_ROUTE && M == 1 && FMT != UT_FMT_F32)
        staged_route = a.plan_ids && a.route_lg && a.x.self_max && !a.x.dig;
    if (staged_route) {
        if constexpr (STAGED_ROUTE && M == 1 && FMT != UT_FMT_F32) {
            if (tile >= a.ntiles) return;
            cnt = gate_up_route_staged<FMT>(a, u, tile, oc, lds, rows, gsc, usc, exl[0], res);
            if (u >= cnt) return;
        }
    } else if (a.plan_ids) {
        // this wave resolves the slot from the ids (loaded ahead of x) while
        // x's loads are in flight; a slot past the count streams x itself in
        // place of weights (valid memory of at least a row's bytes: f32 x,
        // or its digit planes) and stores nothing
        if (tile >= a.ntiles) return;
        const int n = a.plan_M * a.plan_k;
        int id = (M > 1 || !a.route_lg) && lane < n ? a.plan_ids[lane] : -1;
        const uint8_t *dummy = a.x.xf   ? (const uint8_t *)a.x.xf
                               : a.x.xh ? (const uint8_t *)a.x.xh
                                        : (const uint8_t *)a.x.dig;
        auto mid = [&]() {
            if constexpr (M == 1) if (a.route_lg) {
                // wave m routes row m; the choices go round through LDS
                __shared__ int32_t s_rid[64];
                __shared__ float s_rw[64];
                if (wave < a.plan_M) {
                    int32_t rid = -1;
                    float rw = 0.0f;
                    route_row_wave<4>(a.route_lg + (int64_t)wave * a.E, a.route_bias, (int)a.E,
                                      a.plan_k, a.route_ng, a.route_tg, a.route_norm,
                                      a.route_scale, &rid, &rw);
                    if (lane < a.plan_k) {
                        s_rid[wave * a.plan_k + lane] = rid;
                        s_rw[wave * a.plan_k + lane] = rw;
                    }
                }
                asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
                id = lane < n ? s_rid[lane] : -1;
                if (u == 0 && tile == 0 && wave == 0 && lane < n) {
                    a.route_ids[lane] = id;
                    a.route_w[lane] = s_rw[lane];
                }
            }
            const void *p6[6];
            cnt = plan_slot_wave(id, n, a.E, a.ptbl, u, u == 0 && tile == 0 && wave == 0, a.plan,
                                 a.err_flag, p6);
            const bool live = u < cnt;
            rows[0] = live ? (const uint8_t *)p6[kSpGate] + oc * a.row_bytes : dummy;
            rows[1] = live ? (const uint8_t *)p6[kSpUp] + oc * a.row_bytes : dummy;
            gsc = live ? (const float *)p6[kSpGateS] : nullptr;
            usc = live ? (const float *)p6[kSpUpS] : nullptr;
        };
        gemv_core<FMT, M, 2, gemv_depth<M>()>(rows, a.H, a.x, lds, res, 0, -1, prep, mid);
        if (u >= cnt || tile >= a.ntiles) return;
    } else {
        // the slot count and the slot's pointers load in parallel
        cnt = *a.count;
        const uint8_t *gw = (const uint8_t *)a.sp[u * 6 + kSpGate];
        const uint8_t *uw = (const uint8_t *)a.sp[u * 6 + kSpUp];
        gsc = (const float *)a.sp[u * 6 + kSpGateS];
        usc = (const float *)a.sp[u * 6 + kSpUpS];
        if (u >= cnt || tile >= a.ntiles) return;
        rows[0] = gw + oc * a.row_bytes;
        rows[1] = uw + oc * a.row_bytes;
        gemv_core<FMT, M, 2, gemv_depth<M>()>(rows, a.H, a.x, lds, res, 0, -1, prep);
    }
#pragma unroll
    for (int m = 0; m < M; m++) {
        // f32: the gate value lives on sub-lane m, the up value on 4 + m
        float gv = 0.0f, uv = 0.0f;
        if constexpr (FMT == UT_FMT_F32) {
            uv = __shfl(res.F[1][m], (lane & ~15) | (4 + m), 64);
            gv = res.F[0][m];
        }
        if (s == m && o < a.I) {
            if constexpr (FMT != UT_FMT_F32) {
                gv = int_total_to_f32(res.S[0][m], exl[m], ld_global_f32(gsc + o));
                uv = int_total_to_f32(res.S[1][m], exl[m], ld_global_f32(usc + o));
            }
            // silu(g) * u (undertow-quant/src/lib.rs:121; model.rs:241-247)
            float sg = gv / (1.0f + expf(-gv));
            float hv = __fmul_rn(sg, uv);
            a.h[((int64_t)u * M + m) * a.I + o] = hv;
            atomicMax(&wg_max[m], __float_as_uint(fabsf(hv)));
        }
    }
    __syncthreads();
    if (tid < M) a.hmax_parts[((int64_t)u * M + tid) * a.ntiles + tile] = wg_max[tid];
}

template <int FMT, int M>
__global__ __launch_bounds__(kGemvThreads) void k_moe_gate_up(GateUpArgs a) {
    __shared__ __attribute__((aligned(16))) uint32_t lds[kLdsWords];
    __shared__ uint32_t wg_max[4];
    gate_up_body<FMT, M>(a, blockIdx.y, blockIdx.x, lds, wg_max);
}

// Gate/up on the matrix cores (int4, 2..4 rows, plan ready, H % 512 == 0):
// each wave TW tiles of 8 h rows (A rows 0-7 the gate rows, 8-15 the up
// rows of one tile), the workgroup 32 * TW rows (2 * TW of the plain
// kernel's 16-row tiles: every partial-max slot gets the workgroup's
// maximum).  x is digitised while staged, by the digitiser's exponents,
// into the same integers as its digit planes; the wave's tiles share each
// staged chunk, so TW = 2 halves the activation staging per weight byte.
template <int M> constexpr int gate_up_mfma_kc() { return M == 2 ? 4096 : 2048; }
// Tiles per wave: two when the routed experts have the launch to
// themselves; in the 2-D grid beside a shared MLP (whose 16-row tiles set
// the grid) one.
template <int M, bool DUAL> constexpr int gate_up_mfma_tw() { return !DUAL && M >= 2 ? 2 : 1; }
// Tiles per wave of the routed experts beside a shared MLP on the flat grid
// (k_moe_gate_up_mfma_dual_flat): two.  With verify rows of distinct tokens
// (about 15 unique experts at two rows, 28 at four) the config-4 launch
// took 52.9 -> 48.0 us at two rows and 87.5 -> 78.8 us at four against one
// tile per wave (one on the flat grid: 52.5 / 86.5 us).
#ifndef UT_GATE_UP_DUAL_TW
#define UT_GATE_UP_DUAL_TW 2
#endif
template <int M, bool DUAL> constexpr int gate_up_mfma_rows() { return 32 * gate_up_mfma_tw<M, DUAL>(); }
// LDS of the matrix-core gate/up: the staged x chunk, then each wave's
// weight-transpose area
template <int M, bool DUAL> constexpr int gate_up_mfma_lds_words() {
    return mfma_lds_words<M, gate_up_mfma_kc<M>()>() + 4 * gate_up_mfma_tw<M, DUAL>() * kI4WaveAreaBytes / 4;
}

template <int M, int TW>
__device__ __forceinline__ void gate_up_mfma_body(const GateUpArgs &a, int u, int tile,
                                                  uint32_t *lds, uint32_t *wg_max) {
    constexpr int KC = gate_up_mfma_kc<M>();
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, s = lane & 15;
    const int cnt = *a.count;
    const uint8_t *gw = (const uint8_t *)a.sp[u * 6 + kSpGate];
    const uint8_t *uw = (const uint8_t *)a.sp[u * 6 + kSpUp];
    const float *gsc = (const float *)a.sp[u * 6 + kSpGateS];
    const float *usc = (const float *)a.sp[u * 6 + kSpUpS];
    clear_arrivals(a, u, tile);
    if (u >= cnt) return;
    if (tid < 4) wg_max[tid] = 0;
    const int64_t o0 = (int64_t)tile * (32 * TW) + wave * (8 * TW);  // tile w: rows o0 + 8w ..
    // tile rows 0-7 are gate rows o0 + 8w .., rows 8-15 the same up rows;
    // load instruction r takes tile row 8r + lane / 8: gate (r = 0) or up
    const uint8_t *lrows[TW][2];
#pragma unroll
    for (int w = 0; w < TW; w++) {
        const int64_t o = o0 + 8 * w + (lane >> 3), ao = o < a.I ? o : a.I - 1;
        lrows[w][0] = gw + ao * a.row_bytes;
        lrows[w][1] = uw + ao * a.row_bytes;
    }
    int32_t exl[M], sh[M];
#pragma unroll
    for (int m = 0; m < M; m++) {
        exl[m] = a.exps[m];
        sh[m] = exl[m] == INT32_MIN ? INT32_MIN : -exl[m];
    }
    CoreOut<UT_FMT_INT4, M, 4> res[TW];
    mfma_gemv_i4_chunks<M, KC, TW>(lrows, a.H, a.mfma_xf, a.H, sh, (uint8_t *)lds,
                                   (uint8_t *)lds + 4 * mfma_lds_words<M, KC>() +
                                       wave * TW * kI4WaveAreaBytes,
                                   res);
    // per tile: lanes 0-31 hold the gate totals of rows 4g + r (g < 2),
    // lanes 32-63 the up totals of the same rows
    const int r = s >> 2, m = s & 3;
    const int32_t e = m == 0 ? exl[0] : m == 1 ? exl[M > 1 ? 1 : 0]
                    : m == 2 ? exl[M > 2 ? 2 : 0] : exl[M > 3 ? 3 : 0];
#pragma unroll
    for (int w = 0; w < TW; w++) {
        const int64_t S = res[w].S[0][0];
        const int lo = (int)(uint32_t)S, hi = (int)(uint32_t)((uint64_t)S >> 32);
        const int ulo = __shfl(lo, lane + 32 < 64 ? lane + 32 : lane, 64);
        const int uhi = __shfl(hi, lane + 32 < 64 ? lane + 32 : lane, 64);
        const int64_t o = o0 + 8 * w + 4 * g + r;
        if (g < 2 && m < M && o < a.I) {
            const int64_t US = (int64_t)(((uint64_t)(uint32_t)uhi << 32) | (uint32_t)ulo);
            const float gv = int_total_to_f32(S, e, ld_global_f32(gsc + o));
            const float uv = int_total_to_f32(US, e, ld_global_f32(usc + o));
            // silu(g) * u (undertow-quant/src/lib.rs:121; model.rs:241-247)
            const float sg = gv / (1.0f + expf(-gv));
            const float hv = __fmul_rn(sg, uv);
            a.h[((int64_t)u * M + m) * a.I + o] = hv;
            atomicMax(&wg_max[m], __float_as_uint(fabsf(hv)));
        }
    }
    __syncthreads();
    if (tid < 2 * TW * M) {
        const int mm = tid / (2 * TW), part = 2 * TW * tile + tid % (2 * TW);
        if (part < a.ntiles) a.hmax_parts[((int64_t)u * M + mm) * a.ntiles + part] = wg_max[mm];
    }
}

template <int M>
__global__ __launch_bounds__(kGemvThreads) void k_moe_gate_up_mfma(GateUpArgs a) {
    __shared__ __attribute__((aligned(16))) uint32_t lds[gate_up_mfma_lds_words<M, false>()];
    __shared__ uint32_t wg_max[4];
    gate_up_mfma_body<M, gate_up_mfma_tw<M, false>()>(a, blockIdx.y, blockIdx.x, lds, wg_max);
}

// Gate/up of int8 experts on the matrix cores (UT_MOE_I8_MFMA_MIN_M..4
// rows, plan ready, x as the digitiser's three base-256 planes, H % 256 ==
// 0): v_mfma_i32_16x16x64_i8 over the weights' own bytes (mfma_gemv_i8).
// Each wave TW tiles of 8 h rows: load instructions 0-1 take the tile's
// gate rows, 2-3 the same up rows, so the totals land as in the int4
// kernel (lanes 0-31 gate, 32-63 up) and its epilogue applies unchanged.
#ifndef UT_MOE_I8_MFMA_DEPTH
#define UT_MOE_I8_MFMA_DEPTH 2
#endif
constexpr int kGateUpI8TW = 1;
constexpr int kMoeI8KC = 2048;
template <int M> constexpr int moe_i8_mfma_lds_bytes(int tw) {
    return mfma_i8_lds_bytes<M, kMoeI8KC>() + 4 * tw * kMfmaI8WaveAreaBytes;
}

template <int M>
__device__ __forceinline__ void gate_up_i8_mfma_body(const GateUpArgs &a, int u, int tile,
                                                     uint8_t *lds, uint32_t *wg_max) {
    constexpr int TW = kGateUpI8TW;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, s = lane & 15;
    const int cnt = *a.count;
    const uint8_t *gw = (const uint8_t *)a.sp[u * 6 + kSpGate];
    const uint8_t *uw = (const uint8_t *)a.sp[u * 6 + kSpUp];
    const float *gsc = (const float *)a.sp[u * 6 + kSpGateS];
    const float *usc = (const float *)a.sp[u * 6 + kSpUpS];
    clear_arrivals(a, u, tile);
    if (u >= cnt) return;
    if (tid < 4) wg_max[tid] = 0;
    const int64_t o0 = (int64_t)tile * (32 * TW) + wave * (8 * TW);
    // instruction r takes tile row 4r + lane / 16: gate rows (r < 2) or up
    const uint8_t *lrows[TW][4];
#pragma unroll
    for (int w = 0; w < TW; w++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int64_t o = o0 + 8 * w + 4 * (r & 1) + (lane >> 4), ao = o < a.I ? o : a.I - 1;
            lrows[w][r] = (r < 2 ? gw : uw) + ao * a.row_bytes;
        }
    int32_t exl[M];
#pragma unroll
    for (int m = 0; m < M; m++) exl[m] = a.exps[m];
    CoreOut<UT_FMT_INT4, M, 4> res[TW];
    mfma_gemv_i8<M, kMoeI8KC, TW, UT_MOE_I8_MFMA_DEPTH, false>(
        lrows, 0, a.H, a.x.dig, a.x.KW, nullptr, 0, lds,
        lds + mfma_i8_lds_bytes<M, kMoeI8KC>() + wave * TW * kMfmaI8WaveAreaBytes, res,
        [](int32_t (&)[4]) {});
    const int r = s >> 2, m = s & 3;
    const int32_t e = m == 0 ? exl[0] : m == 1 ? exl[M > 1 ? 1 : 0]
                    : m == 2 ? exl[M > 2 ? 2 : 0] : exl[M > 3 ? 3 : 0];
#pragma unroll
    for (int w = 0; w < TW; w++) {
        const int64_t S = res[w].S[0][0];
        const int lo = (int)(uint32_t)S, hi = (int)(uint32_t)((uint64_t)S >> 32);
        const int ulo = __shfl(lo, lane + 32 < 64 ? lane + 32 : lane, 64);
        const int uhi = __shfl(hi, lane + 32 < 64 ? lane + 32 : lane, 64);
        const int64_t o = o0 + 8 * w + 4 * g + r;
        if (g < 2 && m < M && o < a.I) {
            const int64_t US = (int64_t)(((uint64_t)(uint32_t)uhi << 32) | (uint32_t)ulo);
            const float gv = int_total_to_f32(S, e, ld_global_f32(gsc + o));
            const float uv = int_total_to_f32(US, e, ld_global_f32(usc + o));
            // silu(g) * u (undertow-quant/src/lib.rs:121; model.rs:241-247)
            const float sg = gv / (1.0f + expf(-gv));
            const float hv = __fmul_rn(sg, uv);
            a.h[((int64_t)u * M + m) * a.I + o] = hv;
            atomicMax(&wg_max[m], __float_as_uint(fabsf(hv)));
        }
    }
    __syncthreads();
    if (tid < 2 * TW * M) {
        const int mm = tid / (2 * TW), part = 2 * TW * tile + tid % (2 * TW);
        if (part < a.ntiles) a.hmax_parts[((int64_t)u * M + mm) * a.ntiles + part] = wg_max[mm];
    }
}

template <int M>
__global__ __launch_bounds__(kGemvThreads) void k_moe_gate_up_i8_mfma(GateUpArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[moe_i8_mfma_lds_bytes<M>(kGateUpI8TW)];
    __shared__ uint32_t wg_max[4];
    gate_up_i8_mfma_body<M>(a, blockIdx.y, blockIdx.x, lds, wg_max);
}

constexpr int cmax_words(int p, int q) { return p > q ? p : q; }

// The routed experts on the matrix cores and a shared MLP of format FB in
// one launch, so the shared MLP's few workgroups run beside the routed ones
// instead of after them, on a flat grid: gxm tiles of 32 * TW rows per
// routed slot (slot-major, nrouted workgroups) and the shared MLP's 16-row
// tiles, so no workgroup of the grid is empty when the routed tiles are
// fewer than the shared MLP's.
// The shared MLP's workgroups first in the dual launches' grids (1), or
// after the routed ones (0).  A shared int8 workgroup streams twice the
// bytes of a routed int4 one; dispatched last, they ran on alone at the
// launch's end: config-4 four-row verify gate/up 79.1 -> 68.4 us, two-row
// 47.7 -> 44.8 us, one-row 30.9 -> 30.2 us.
#ifndef UT_DUAL_SHARED_FIRST
#define UT_DUAL_SHARED_FIRST 1
#endif
template <int M, int FB, int TW>
__global__ __launch_bounds__(kGemvThreads) void k_moe_gate_up_mfma_dual_flat(GateUpArgs a,
                                                                             GateUpArgs b, int gxm,
                                                                             int nrouted) {
    __shared__ __attribute__((aligned(16)))
    uint32_t lds[cmax_words(mfma_lds_words<M, gate_up_mfma_kc<M>()>() + TW * kI4WaveAreaBytes,
                            kLdsWords)];
    __shared__ uint32_t wg_max[4];
    const int nb = gridDim.x - nrouted;
    const int i = UT_DUAL_SHARED_FIRST ? (blockIdx.x < nb ? nrouted + blockIdx.x : blockIdx.x - nb)
                                       : blockIdx.x;
    if (i < nrouted) gate_up_mfma_body<M, TW>(a, i / gxm, i % gxm, lds, wg_max);
    else gate_up_body<FB, M, false>(b, 0, i - nrouted, lds, wg_max);
}

// Routed experts (format FA) and one shared MLP (format FB) in one launch:
// grid rows are the routed slots and the shared MLP's row (the first with
// UT_DUAL_SHARED_FIRST, else the last).
template <int FA, int FB, int M>
// At one and two rows, registers for five workgroups per CU (a few spilled
// values): at one row the routed and shared experts' 9 x 128 workgroups are
// then all resident at once (four per CU left 128 for a second pass:
// 32.6 -> 29.9 us), at two rows the 17 x 128 take 1.7 passes instead of 2.1
// (66.9 -> 63.4 us).  The plain kernel's 1,024 workgroups at one row need
// only four per CU and run faster without the bound's spills.
__global__ __launch_bounds__(kGemvThreads, M <= 2 ? 5 : 1) void k_moe_gate_up_dual(GateUpArgs a, GateUpArgs b) {
    __shared__ __attribute__((aligned(16))) uint32_t lds[kLdsWords];
    __shared__ uint32_t wg_max[4];
    // (the routed table's x comes digitised here: no staged routing)
    const int y = UT_DUAL_SHARED_FIRST ? (blockIdx.y == 0 ? gridDim.y - 1 : blockIdx.y - 1)
                                       : blockIdx.y;
    if (y + 1 < gridDim.y)
        gate_up_body<FA, M, false>(a, y, blockIdx.x, lds, wg_max);
    else
        gate_up_body<FB, M, false>(b, 0, blockIdx.x, lds, wg_max);
}

// --------------------------------------------------------------- down ---
// The routed experts' combine folded into down: each workgroup of a row
// band (one per slot) stores its d rows device-coherently and counts in at
// arrive[band]; the one that counts last adds the band's columns of out as
// k_moe_combine4 does (router choice order, the same init / extra /
// shared / accumulate terms), so no combine launch follows.  The counters
// are cleared by the gate/up launch before (GateUpArgs::arrive).
struct CombineFold {
    int32_t *arrive = nullptr;  // [bands]; nullptr: no fold
    const int32_t *choice_slot = nullptr;
    const float *weights = nullptr;
    int k = 0, extra = 0, accumulate = 0;
    const float *dshared = nullptr, *init = nullptr;
    float *out = nullptr;
    int64_t ldo = 0;
};

struct DownArgs {
    ExpertPtrs tbl;
    const void *const *sp;  // the plan's per-slot weight pointers
    const int32_t *uniq;
    const int32_t *count;
    int64_t H, I, row_bytes;  // down is [H, I]
    XSrc x;                   // h (f32, digitised while staged): slot u's rows start at u*M
    int64_t x_slot_stride;    // floats between slots
    const uint32_t *hmax_parts;  // [slots*M][nparts] max|h| bits from the gate/up kernel
    int nparts;
    float *d;                 // [slots][M][H]
    // split-K over blockIdx.z (ks > 1, one-slot MLPs): columns
    // [z*kslice, (z+1)*kslice), exact partial totals to part[z][slot][M][H]
    // (f32 weights: the partial's bits), finished by k_moe_down_finish
    int ks = 1;
    int64_t kslice = 0;
    int64_t *part = nullptr;
    CombineFold fold{};
};

template <int M>
__device__ void fold_combine(const DownArgs &a, int band, int64_t c0, int ncols);

// A finished d value.  With the combine folded into the launch it is
// stored device-coherently (a relaxed agent-scope atomic store, written
// through this XCD's L2), so the band's last workgroup, on any XCD, reads
// it without a cache write-back.
__device__ __forceinline__ void store_d(const DownArgs &a, int64_t i, float v) {
    if (UT_MOE_FOLD_COMBINE && a.fold.arrive)
        __hip_atomic_store(a.d + i, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
        a.d[i] = v;
}

// The digitisation shift of h row (u, m): 22 - E with max|h| < 2^E, from the
// gate/up workgroups' partial maxima (INT32_MIN: non-finite row).  Whole
// workgroup; red4: 4 words of LDS.
__device__ __forceinline__ int32_t h_shift(const uint32_t *hmax_parts, int nparts, int64_t row,
                                           uint32_t *red4) {
    return rowmax_shift(hmax_parts, nparts, row, red4);
}

// Rows per lane: 2 (registers for three or four workgroups per CU; at M = 1
// also every weight step in flight; four rows per lane at M = 2 held two
// workgroups per CU and measured slower).
template <int M> constexpr int down_rows() { return 2; }

// Staged columns of down's h: inter sizes up to 2048 stage once (fewer
// staging registers, so more workgroups fit a CU); longer K is staged in
// chunks, or split (one-slot MLPs, kslice <= this).
template <int FMT, int M> constexpr int down_kc() { return gemv_chunk_cols<FMT, M, 2048>(); }

// Weight steps in flight in down: at M = 1 four (all of a 2048-column
// int4 row), two at M = 2, else the core's default.
template <int M> constexpr int down_depth() { return M == 1 ? 4 : M == 2 ? 2 : gemv_depth<M>(); }

template <int FMT, int M>
__device__ __forceinline__ void down_body(const DownArgs &a, int u, int tile, uint32_t *lds) {
    constexpr int R = down_rows<M>();
    const int cnt = *a.count;
    const uint8_t *dw = (const uint8_t *)a.sp[u * 6 + kSpDown];
    const float *dsc = (const float *)a.sp[u * 6 + kSpDownS];
    if (u >= cnt) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, s = lane & 15;
    const int64_t row0 = (int64_t)tile * (16 * R) + wave * (4 * R) + g * R;
    const uint8_t *rows[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        int64_t o = row0 + r < a.H ? row0 + r : a.H - 1;
        rows[r] = dw + o * a.row_bytes;
    }
    XSrc xs = a.x;
    xs.xf = a.x.xf + u * a.x_slot_stride;
    xs.dig = nullptr;
    int32_t exl[M];
    const int64_t kb = a.ks > 1 ? (int64_t)blockIdx.z * a.kslice : 0;
    const int64_t ke = a.ks > 1 ? (kb + a.kslice < a.I ? kb + a.kslice : a.I) : a.I;
    // the row exponents of h from the gate/up workgroups' partial maxima:
    // their loads go out first; on the one-chunk path the reduction runs
    // inside the staging, after the first weight loads (prep)
    __shared__ uint32_t red[4 * M];
    ut_u32x4 pv[M];
    constexpr int KC = down_kc<FMT, M>();
    const bool late = FMT != UT_FMT_F32 && gemv_one_chunk<FMT, M, KC>(kb, ke);
    if constexpr (FMT != UT_FMT_F32) {
        rowmax_load<M>(a.hmax_parts + (int64_t)u * M * a.nparts, a.nparts, pv);
        if (!late) {
            int32_t sh[M];
            rowmax_reduce<M>(pv, sh, red);
#pragma unroll
            for (int m = 0; m < M; m++) {
                xs.sh[m] = sh[m];
                exl[m] = sh[m] == INT32_MIN ? INT32_MIN : -sh[m];
            }
        }
    }
    auto prep = [&](int32_t (&shl)[4]) {
        if constexpr (FMT != UT_FMT_F32) {
            int32_t sh[M];
            rowmax_reduce<M>(pv, sh, red);
#pragma unroll
            for (int m = 0; m < M; m++) {
                shl[m] = sh[m];
                exl[m] = sh[m] == INT32_MIN ? INT32_MIN : -sh[m];
            }
        }
    };
    CoreOut<FMT, M, R> res;
    if (a.ks > 1) {
        gemv_core<FMT, M, R, down_depth<M>(), KC>(rows, a.I, xs, lds, res, kb, ke, prep);
        const int64_t slots = gridDim.y;
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int m = 0; m < M; m++) {
                const int64_t o = row0 + r;
                if (s == 4 * r + m && o < a.H)
                    a.part[(((int64_t)blockIdx.z * slots + u) * M + m) * a.H + o] =
                        FMT == UT_FMT_F32 ? (int64_t)__float_as_uint(res.F[r][m]) : res.S[r][m];
            }
        return;
    }
    gemv_core<FMT, M, R, down_depth<M>(), KC>(rows, a.I, xs, lds, res, 0, -1, prep);
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int m = 0; m < M; m++) {
            const int64_t o = row0 + r;
            if (s == 4 * r + m && o < a.H) {
                float v = core_value<FMT, M, R>(res, r, m, exl, dsc, o);
                store_d(a, ((int64_t)u * M + m) * a.H + o, v);
            }
        }
}

// Down on the matrix cores (int4, 2..4 rows, the inter size staged whole:
// I <= 2048, I % 128 == 0, no split): each wave TW x 16 rows, the
// workgroup 64 TW;
// the same totals and epilogue as down_body.
// UT_DOWN_MFMA_MIN_M: the fewest rows that take it (experiments).
#ifndef UT_DOWN_MFMA_MIN_M
#define UT_DOWN_MFMA_MIN_M 2
#endif
#ifndef UT_DOWN_MFMA_DEPTH
#define UT_DOWN_MFMA_DEPTH 4
#endif
template <int M> constexpr int down_mfma_depth() { return UT_DOWN_MFMA_DEPTH; }
// 16-row tiles per wave (one staged h for TW x 16 rows): two from three
// rows on (C2 down at four rows 69.3 -> 67.0 us), one at two rows (two
// measured 29.2 -> 32.7 us there)
#ifndef UT_DOWN_MFMA_TW
#define UT_DOWN_MFMA_TW (M >= 3 ? 2 : 1)
#endif
template <int M> constexpr int down_mfma_tw() { return UT_DOWN_MFMA_TW; }
constexpr int kDownMfmaKC = 2048;
inline bool down_mfma_ok(int fmt, int M, int64_t I, int ks) {
    return fmt == UT_FMT_INT4 && M >= UT_DOWN_MFMA_MIN_M && M <= 4 && ks == 1 &&
           I <= kDownMfmaKC && I % kMfmaStepCols == 0;
}

template <int M>
__device__ __forceinline__ void down_mfma_body(const DownArgs &a, int u, int tile, uint32_t *lds,
                                               uint32_t *red) {
    if (u >= *a.count) return;
    const uint8_t *dw = (const uint8_t *)a.sp[u * 6 + kSpDown];
    const float *dsc = (const float *)a.sp[u * 6 + kSpDownS];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, s = lane & 15;
    constexpr int TW = down_mfma_tw<M>();
    const int64_t wrow0 = (int64_t)tile * (64 * TW) + wave * (16 * TW);
    // load instruction r of tile w takes tile row 8r + lane / 8
    const uint8_t *lrows[TW][2];
#pragma unroll
    for (int w = 0; w < TW; w++)
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int64_t o = wrow0 + 16 * w + 8 * r + (lane >> 3);
            lrows[w][r] = dw + (o < a.H ? o : a.H - 1) * a.row_bytes;
        }
    ut_u32x4 pv[M];
    rowmax_load<M>(a.hmax_parts + (int64_t)u * M * a.nparts, a.nparts, pv);
    int32_t exl[M];
    auto prep = [&](int32_t (&shl)[4]) {
        int32_t sh[M];
        rowmax_reduce<M>(pv, sh, red);
#pragma unroll
        for (int m = 0; m < M; m++) {
            shl[m] = sh[m];
            exl[m] = sh[m] == INT32_MIN ? INT32_MIN : -sh[m];
        }
    };
    CoreOut<UT_FMT_INT4, M, 4> res[TW];
    mfma_gemv_i4_f32x<M, down_mfma_depth<M>() / 2, kDownMfmaKC, TW>(
        lrows, a.I, a.x.xf + u * a.x_slot_stride, a.x.ldx, (uint8_t *)lds,
        (uint8_t *)lds + 4 * mfma_lds_words<M, kDownMfmaKC>() + wave * TW * kI4WaveAreaBytes, res,
        prep);
#pragma unroll
    for (int w = 0; w < TW; w++)
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int m = 0; m < M; m++) {
                const int64_t o = wrow0 + 16 * w + 4 * g + r;
                if (s == 4 * r + m && o < a.H)
                    store_d(a, ((int64_t)u * M + m) * a.H + o,
                            core_value<UT_FMT_INT4, M, 4>(res[w], r, m, exl, dsc, o));
            }
}

// LDS of the matrix-core down: the staged h, then each wave's
// weight-transpose area
template <int M> constexpr int down_mfma_lds_words() {
    return mfma_lds_words<M, kDownMfmaKC>() + 4 * down_mfma_tw<M>() * kI4WaveAreaBytes / 4;
}

template <int M>
__global__ __launch_bounds__(kGemvThreads) void k_moe_down_mfma(DownArgs a) {
    __shared__ __attribute__((aligned(16))) uint32_t lds[down_mfma_lds_words<M>()];
    __shared__ uint32_t red[4 * M];
    down_mfma_body<M>(a, blockIdx.y, blockIdx.x, lds, red);
    if (UT_MOE_FOLD_COMBINE && a.fold.arrive) fold_combine<M>(a, blockIdx.x, (int64_t)blockIdx.x * 64 * down_mfma_tw<M>(),
                                       64 * down_mfma_tw<M>());
}

// Down of int8 experts on the matrix cores (UT_MOE_I8_MFMA_MIN_M..4 rows,
// I <= 2048 staged whole, I % 256 == 0, no split): h as f32 digitised while
// staged by the gate/up workgroups' partial maxima, each wave one 16-row
// tile, the workgroup 64 rows; the same totals and epilogue as down_body.
// Whole 256-column segments in every K slice, each slice staged in one
// chunk: the inter size whole (ks == 1) or split in slices of kslice
// columns (a one-slot MLP's down, finished by k_moe_down_finish).
inline bool down_i8_mfma_ok(int fmt, int M, int64_t I, int ks, int64_t kslice) {
    if (fmt != UT_FMT_INT8 || M < UT_MOE_I8_MFMA_MIN_M || M > 4 || I % kMfmaI8SegCols != 0)
        return false;
    if (ks == 1) return I <= kMoeI8KC;
    return kslice <= kMoeI8KC && kslice % kMfmaI8SegCols == 0;
}

template <int M>
__global__ __launch_bounds__(kGemvThreads) void k_moe_down_i8_mfma(DownArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[moe_i8_mfma_lds_bytes<M>(1)];
    __shared__ uint32_t red[4 * M];
    const int u = blockIdx.y, tile = blockIdx.x;
    if (u < *a.count) {
        const uint8_t *dw = (const uint8_t *)a.sp[u * 6 + kSpDown];
        const float *dsc = (const float *)a.sp[u * 6 + kSpDownS];
        const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, s = lane & 15;
        const int64_t wrow0 = (int64_t)tile * 64 + wave * 16;
        // instruction r takes tile row 4r + lane / 16
        const uint8_t *lrows[1][4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int64_t o = wrow0 + 4 * r + (lane >> 4);
            lrows[0][r] = dw + (o < a.H ? o : a.H - 1) * a.row_bytes;
        }
        ut_u32x4 pv[M];
        rowmax_load<M>(a.hmax_parts + (int64_t)u * M * a.nparts, a.nparts, pv);
        int32_t exl[M];
        auto prep = [&](int32_t (&shl)[4]) {
            int32_t sh[M];
            rowmax_reduce<M>(pv, sh, red);
#pragma unroll
            for (int m = 0; m < M; m++) {
                shl[m] = sh[m];
                exl[m] = sh[m] == INT32_MIN ? INT32_MIN : -sh[m];
            }
        };
        CoreOut<UT_FMT_INT4, M, 4> res[1];
        // split K (ks > 1): columns [z kslice, (z+1) kslice), exact partial
        // totals to part[z][slot][M][H] as down_body writes them
        const int64_t kb = a.ks > 1 ? (int64_t)blockIdx.z * a.kslice : 0;
        const int64_t ke = a.ks > 1 ? (kb + a.kslice < a.I ? kb + a.kslice : a.I) : a.I;
        mfma_gemv_i8<M, kMoeI8KC, 1, UT_MOE_I8_MFMA_DEPTH, true>(
            lrows, kb, ke, nullptr, 0, a.x.xf + u * a.x_slot_stride, a.x.ldx, lds,
            lds + mfma_i8_lds_bytes<M, kMoeI8KC>() + wave * kMfmaI8WaveAreaBytes, res, prep);
        if (a.ks > 1) {
            const int64_t slots = gridDim.y;
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int m = 0; m < M; m++) {
                    const int64_t o = wrow0 + 4 * g + r;
                    if (s == 4 * r + m && o < a.H)
                        a.part[(((int64_t)blockIdx.z * slots + u) * M + m) * a.H + o] =
                            res[0].S[r][m];
                }
            return;
        }
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int m = 0; m < M; m++) {
                const int64_t o = wrow0 + 4 * g + r;
                if (s == 4 * r + m && o < a.H)
                    store_d(a, ((int64_t)u * M + m) * a.H + o,
                            int_total_to_f32(res[0].S[r][m], exl[m], ld_global_f32(dsc + o)));
            }
    }
    if (UT_MOE_FOLD_COMBINE && a.fold.arrive) fold_combine<M>(a, blockIdx.x, (int64_t)blockIdx.x * 64, 64);
}

// The routed experts' down on the matrix cores and a shared MLP's down
// (format FB, one slot, no split) in one launch: a flat grid of gxm tiles
// per routed slot (slot-major, as k_moe_down_mfma's grid) and the shared
// MLP's gxb tiles (first with UT_DUAL_SHARED_FIRST), which run beside the
// routed ones instead of after them.
template <int M, int FB>
__global__ __launch_bounds__(kGemvThreads) void k_moe_down_mfma_dual(DownArgs a, DownArgs b, int gxm,
                                                                    int nrouted) {
    __shared__ __attribute__((aligned(16)))
    uint32_t lds[cmax_words(down_mfma_lds_words<M>(), kLdsWords)];
    __shared__ uint32_t red[4 * M];
    const int nb = gridDim.x - nrouted;
    const int i = UT_DUAL_SHARED_FIRST ? (blockIdx.x < nb ? nrouted + blockIdx.x : blockIdx.x - nb)
                                       : blockIdx.x;
    if (i < nrouted) down_mfma_body<M>(a, i / gxm, i % gxm, lds, red);
    else down_body<FB, M>(b, 0, i - nrouted, lds);
}

template <int FMT, int M>
__global__ __launch_bounds__(kGemvThreads) void k_moe_down(DownArgs a) {
    __shared__ __attribute__((aligned(16))) uint32_t lds[kLdsWords];
    down_body<FMT, M>(a, blockIdx.y, blockIdx.x, lds);
    if (UT_MOE_FOLD_COMBINE && a.fold.arrive) {
        constexpr int DR = 16 * down_rows<M>();
        fold_combine<M>(a, blockIdx.x, (int64_t)blockIdx.x * DR, DR);
    }
}

// Sums the split-K partials of down (slot u, row m) in z order (integers
// exactly, f32 in that fixed order) and applies the row epilogue into d.
// Grid (H / 256, slots * M).
template <int FMT>
__global__ __launch_bounds__(kGemvThreads) void k_moe_down_finish(DownArgs a, int M) {
    __shared__ uint32_t red4[4];
    const int u = blockIdx.y / M, m = blockIdx.y - u * M;
    if (u >= *a.count) return;
    int32_t exl = 0;
    if constexpr (FMT != UT_FMT_F32) {
        const int32_t sh = h_shift(a.hmax_parts, a.nparts, (int64_t)u * M + m, red4);
        exl = sh == INT32_MIN ? INT32_MIN : -sh;
    }
    const int64_t o = (int64_t)blockIdx.x * kGemvThreads + threadIdx.x;
    if (o >= a.H) return;
    const int64_t slots = gridDim.y / M;
    const int64_t zs = slots * M * a.H;
    const int64_t i = ((int64_t)u * M + m) * a.H + o;
    float v;
    if constexpr (FMT == UT_FMT_F32) {
        v = __uint_as_float((uint32_t)a.part[i]);
        for (int z = 1; z < a.ks; z++) v = __fadd_rn(v, __uint_as_float((uint32_t)a.part[z * zs + i]));
    } else {
        int64_t S = a.part[i];
        for (int z = 1; z < a.ks; z++) S += a.part[z * zs + i];
        v = int_total_to_f32(S, exl, ld_global_f32((const float *)a.sp[u * 6 + kSpDownS] + o));
    }
    a.d[i] = v;
}

template <int FA, int FB, int M>
__global__ __launch_bounds__(kGemvThreads) void k_moe_down_dual(DownArgs a, DownArgs b) {
    __shared__ __attribute__((aligned(16))) uint32_t lds[kLdsWords];
    const int y = UT_DUAL_SHARED_FIRST ? (blockIdx.y == 0 ? gridDim.y - 1 : blockIdx.y - 1)
                                       : blockIdx.y;
    if (y + 1 < gridDim.y) down_body<FA, M>(a, y, blockIdx.x, lds);
    else down_body<FB, M>(b, 0, blockIdx.x, lds);
}

// ------------------------------------------------------------ combine ---
// out[s, o] = sum_c w[s,c] * d[slot(s,c), s, o], in router choice order from
// zero (model.rs:268-281: moe_out starts zeroed; the reference adds
// w*d per choice) or from init[s, o].  extra >= 0: then += d[extra, s, o]
// (a dense MLP slot, MlpWeights::forward_add, model.rs:282-284).
// accumulate: out += result.
__global__ void k_moe_combine(const int32_t *__restrict__ choice_slot,
                              const float *__restrict__ weights, const float *__restrict__ d,
                              int M, int k, int64_t H, const int32_t *__restrict__ count,
                              int extra, const float *__restrict__ dshared,
                              const float *__restrict__ init, float *__restrict__ out,
                              int64_t ldo, int accumulate) {
    const int s = blockIdx.y;
    const int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (o >= H) return;
    float acc = init ? init[s * ldo + o] : 0.0f;
#pragma unroll 8
    for (int c = 0; c < k; c++) {
        int slot = choice_slot[s * k + c];
        if (slot < 0) continue;
        acc = __fadd_rn(acc, __fmul_rn(weights[s * k + c], d[((int64_t)slot * M + s) * H + o]));
    }
    if (extra) {
        int slot = *count - 1;
        acc = __fadd_rn(acc, d[((int64_t)slot * M + s) * H + o]);
    }
    // a shared MLP run beside the routed experts (MlpWeights::forward_add
    // after the routed sum, model.rs:282-284)
    if (dshared) acc = __fadd_rn(acc, dshared[(int64_t)s * H + o]);
    float *po = out + s * ldo + o;
    *po = accumulate ? __fadd_rn(*po, acc) : acc;
}

// NC consecutive columns c0.. of row s of k_moe_combine's result, with
// every load issued before the first sum (1 <= k <= 8: the choices' rows
// load in one round trip; an invalid choice reads slot 0's row and is
// skipped), and the sums in k_moe_combine's order.  16-byte aligned rows.
// COH: d was written in the same launch by other workgroups (store_d), so
// its values are read device-coherently (relaxed agent-scope atomic loads).
template <int NC, bool COH = false>
__device__ __forceinline__ void combine_cols(const int32_t *__restrict__ choice_slot,
                                             const float *__restrict__ weights,
                                             const float *__restrict__ d, int M, int k, int64_t H,
                                             const int32_t *__restrict__ count, int extra,
                                             const float *__restrict__ dshared,
                                             const float *__restrict__ init, const float *prev,
                                             int s, int64_t c0, float (&acc)[NC]) {
    constexpr int KF = 8;
    auto ldv = [](const float *p, float (&r)[NC]) {
#pragma unroll
        for (int q = 0; q < NC / 4; q++) {
            const float4 v = *(const float4 *)(p + 4 * q);
            r[4 * q] = v.x; r[4 * q + 1] = v.y; r[4 * q + 2] = v.z; r[4 * q + 3] = v.w;
        }
    };
    auto ldd = [&](const float *p, float (&r)[NC]) {
        if constexpr (COH) {
#pragma unroll
            for (int j = 0; j < NC; j++)
                r[j] = __hip_atomic_load(p + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            ldv(p, r);
        }
    };
    const bool fast = k >= 1 && k <= KF;
    int slot[KF];
    float wc[KF], dv[KF][NC], ex[NC], sh[NC], pv[NC];
    if (fast) {
        // straight-line loads (choices past k repeat the last one, unused)
#pragma unroll
        for (int c = 0; c < KF; c++) {
            const int cc = c < k ? c : k - 1;
            slot[c] = choice_slot[s * k + cc];
            wc[c] = weights[s * k + cc];
        }
#pragma unroll
        for (int c = 0; c < KF; c++)
            ldd(d + ((int64_t)(slot[c] > 0 ? slot[c] : 0) * M + s) * H + c0, dv[c]);
    }
    if (init) ldv(init, acc);
    else
#pragma unroll
        for (int j = 0; j < NC; j++) acc[j] = 0.0f;
    if (extra) ldd(d + ((int64_t)(*count - 1) * M + s) * H + c0, ex);
    if (dshared) ldv(dshared + (int64_t)s * H + c0, sh);
    if (prev) ldv(prev, pv);
    if (fast) {
#pragma unroll
        for (int c = 0; c < KF; c++)
            if (c < k && slot[c] >= 0)
#pragma unroll
                for (int j = 0; j < NC; j++) acc[j] = __fadd_rn(acc[j], __fmul_rn(wc[c], dv[c][j]));
    } else {
        for (int c = 0; c < k; c++) {
            const int sl = choice_slot[s * k + c];
            if (sl < 0) continue;
            float t[NC];
            ldd(d + ((int64_t)sl * M + s) * H + c0, t);
            const float w = weights[s * k + c];
#pragma unroll
            for (int j = 0; j < NC; j++) acc[j] = __fadd_rn(acc[j], __fmul_rn(w, t[j]));
        }
    }
    if (extra)
#pragma unroll
        for (int j = 0; j < NC; j++) acc[j] = __fadd_rn(acc[j], ex[j]);
    if (dshared)
#pragma unroll
        for (int j = 0; j < NC; j++) acc[j] = __fadd_rn(acc[j], sh[j]);
    if (prev)
#pragma unroll
        for (int j = 0; j < NC; j++) acc[j] = __fadd_rn(pv[j], acc[j]);
}

// k_moe_combine with four columns per thread (H % 4 == 0, 16-byte aligned
// rows).
__global__ __launch_bounds__(256) void k_moe_combine4(
    const int32_t *__restrict__ choice_slot, const float *__restrict__ weights,
    const float *__restrict__ d, int M, int k, int64_t H, const int32_t *__restrict__ count,
    int extra, const float *__restrict__ dshared, const float *__restrict__ init,
    float *__restrict__ out, int64_t ldo, int accumulate) {
    const int s = blockIdx.y;
    const int64_t c0 = 4 * ((int64_t)blockIdx.x * blockDim.x + threadIdx.x);
    if (c0 >= H) return;
    float *po = out + s * ldo + c0;
    float acc[4];
    combine_cols<4>(choice_slot, weights, d, M, k, H, count, extra, dshared,
                    init ? init + s * ldo + c0 : nullptr, accumulate ? po : nullptr, s, c0, acc);
    *(float4 *)po = make_float4(acc[0], acc[1], acc[2], acc[3]);
}

// Down's folded combine (CombineFold): columns [c0, c0 + ncols) of every
// row, by the band's last workgroup.  Each thread's d values were stored
// device-coherently (store_d); the thread waits until its stores are
// acknowledged before the workgroup counts in, and the last workgroup reads
// d device-coherently, so no fence writes back or invalidates an L2.
template <int M>
__device__ void fold_combine(const DownArgs &a, int band, int64_t c0, int ncols) {
    __shared__ int s_last;
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
        s_last = __hip_atomic_fetch_add(a.fold.arrive + band, 1, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT) == (int)gridDim.y - 1;
    __syncthreads();
    if (!s_last) return;
    const CombineFold &f = a.fold;
    const int per_row = ncols / 4;
    for (int t = threadIdx.x; t < M * per_row; t += blockDim.x) {
        const int s = t / per_row;
        const int64_t c = c0 + 4 * (t - s * per_row);
        if (c >= a.H) continue;
        float *po = f.out + s * f.ldo + c;
        float acc[4];
        combine_cols<4, true>(f.choice_slot, f.weights, a.d, M, f.k, a.H, a.count, f.extra,
                              f.dshared, f.init ? f.init + s * f.ldo + c : nullptr,
                              f.accumulate ? po : nullptr, s, c, acc);
        *(float4 *)po = make_float4(acc[0], acc[1], acc[2], acc[3]);
    }
}

// The same combine for one row per workgroup (thread t: columns 8t..8t+7,
// each computed exactly as k_moe_combine does), then the finished row
// rms-normalised and digitised by the row digitiser's body (nd: K = H).
__global__ __launch_bounds__(1024) void k_moe_combine_norm(
    const int32_t *__restrict__ choice_slot, const float *__restrict__ weights,
    const float *__restrict__ d, int M, int k, int64_t H, const int32_t *__restrict__ count,
    int extra, const float *__restrict__ dshared, const float *__restrict__ init,
    float *__restrict__ out, int64_t ldo, int accumulate, RowDigArgs nd) {
    __shared__ double redd[16];
    __shared__ uint32_t redu[16];
    const int s = blockIdx.x, tid = threadIdx.x;
    const int64_t c0 = 8 * (int64_t)tid;
    float v[1][8], wv[1][8];
    if (c0 < H) {
        float *po = out + s * ldo + c0;
        const float4 w0 = *(const float4 *)(nd.norm_w + c0), w1 = *(const float4 *)(nd.norm_w + c0 + 4);
        float acc[8];
        combine_cols<8>(choice_slot, weights, d, M, k, H, count, extra, dshared,
                        init ? init + s * ldo + c0 : nullptr, accumulate ? po : nullptr, s, c0, acc);
        wv[0][0] = w0.x; wv[0][1] = w0.y; wv[0][2] = w0.z; wv[0][3] = w0.w;
        wv[0][4] = w1.x; wv[0][5] = w1.y; wv[0][6] = w1.z; wv[0][7] = w1.w;
#pragma unroll
        for (int j = 0; j < 8; j++) v[0][j] = acc[j];
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++) v[0][j] = 0.0f, wv[0][j] = 0.0f;
    }
    // the combined row goes to out after the reductions (nd.raw)
    rowdig_body<1, true>(nd, s, v, wv, redd, redu);
}

bool moe_combine_norm_ok(int64_t H) { return H % 8 == 0 && H <= 8 * 1024; }

// ------------------------------------------------------------- driver ---
size_t moe_scratch_bytes(int64_t M, int64_t k, int64_t slots, int64_t H, int64_t I, int fmt) {
    ScratchLayout L = moe_layout(M, k, slots, H, I, fmt);
    return L.total;
}

ScratchLayout moe_layout(int64_t M, int64_t k, int64_t slots, int64_t H, int64_t I, int fmt) {
    ScratchLayout L;
    auto take = [&](size_t bytes) { size_t off = L.total; L.total += (bytes + 255) & ~size_t(255); return off; };
    const int xflags = fmt == UT_FMT_F32 ? 0 : xdigit_flags_for(fmt, H);
    const int hflags = fmt == UT_FMT_F32 ? 0 : xdigit_flags_for(fmt, I);
    const int64_t ntiles = (I + kGateUpRowsPerWG - 1) / kGateUpRowsPerWG;
    L.count = take(4);
    L.uniq = take((size_t)slots * 4);
    L.choice = take((size_t)M * k * 4);
    L.sp = take((size_t)slots * 6 * sizeof(void *));
    L.xd = take(fmt == UT_FMT_F32 ? 0 : xdigits_bytes(M, H, xflags));
    L.h = take((size_t)slots * M * I * 4);
    L.hmax = take((size_t)slots * M * ntiles * 4);
    L.hd = take(fmt == UT_FMT_F32 ? 0 : xdigits_bytes(slots * M, I, hflags));
    L.d = take((size_t)slots * M * H * 4);
    L.dpart = take(slots == 1 ? (size_t)kDownMaxSplit * M * H * 8 : 0);
    L.xw = take((size_t)M * H * 4);
    L.arrive = take((size_t)(H + 31) / 32 * 4);
    L.xflags = xflags;
    L.hflags = hflags;
    L.ntiles = ntiles;
    return L;
}

template <int FA, int M>
static void launch_gate_up(ut_ctx *ctx, const GateUpArgs &a, int64_t slots, const GateUpArgs *b,
                           int fb) {
    if constexpr (FA == UT_FMT_INT4 && M >= 2 && M <= 4) {
        if (a.mfma_xf) {
            if (!b) {
                constexpr int R = gate_up_mfma_rows<M, false>();
                const unsigned gx = (unsigned)((a.I + R - 1) / R);
                hipLaunchKernelGGL((k_moe_gate_up_mfma<M>), dim3(gx, (unsigned)slots),
                                   dim3(kGemvThreads), 0, ctx->stream, a);
                return;
            }
            // a shared MLP beside it: a flat grid, the routed slots' tiles
            // (UT_GATE_UP_DUAL_TW per wave) and then the shared MLP's
            constexpr int TW = UT_GATE_UP_DUAL_TW;
            constexpr int R = 32 * TW;
            const int gxm = (int)((a.I + R - 1) / R);
            const int nrouted = gxm * (int)slots;
            const dim3 grid((unsigned)(nrouted + b->ntiles));
            if (fb == UT_FMT_INT4)
                hipLaunchKernelGGL((k_moe_gate_up_mfma_dual_flat<M, UT_FMT_INT4, TW>), grid,
                                   dim3(kGemvThreads), 0, ctx->stream, a, *b, gxm, nrouted);
            else
                hipLaunchKernelGGL((k_moe_gate_up_mfma_dual_flat<M, UT_FMT_INT8, TW>), grid,
                                   dim3(kGemvThreads), 0, ctx->stream, a, *b, gxm, nrouted);
            return;
        }
    }
    if constexpr (FA == UT_FMT_INT8 && M >= 2 && M <= 4) {
        if (a.mfma8 && !b) {
            constexpr int R = 32 * kGateUpI8TW;
            const unsigned gx = (unsigned)((a.I + R - 1) / R);
            hipLaunchKernelGGL((k_moe_gate_up_i8_mfma<M>), dim3(gx, (unsigned)slots),
                               dim3(kGemvThreads), 0, ctx->stream, a);
            return;
        }
    }
    if (!b) {
        hipLaunchKernelGGL((k_moe_gate_up<FA, M>), dim3((unsigned)a.ntiles, (unsigned)slots),
                           dim3(kGemvThreads), 0, ctx->stream, a);
        return;
    }
    if constexpr (FA != UT_FMT_F32) {
        const dim3 grid((unsigned)(a.ntiles > b->ntiles ? a.ntiles : b->ntiles), (unsigned)(slots + 1));
        if (fb == UT_FMT_INT4)
            hipLaunchKernelGGL((k_moe_gate_up_dual<FA, UT_FMT_INT4, M>), grid, dim3(kGemvThreads), 0, ctx->stream, a, *b);
        else
            hipLaunchKernelGGL((k_moe_gate_up_dual<FA, UT_FMT_INT8, M>), grid, dim3(kGemvThreads), 0, ctx->stream, a, *b);
    }
}

template <int FA, int M>
static void launch_down(ut_ctx *ctx, const DownArgs &a, int64_t slots, const DownArgs *b, int fb) {
    constexpr int DR = 16 * down_rows<M>();
    const unsigned gx = (unsigned)((a.H + DR - 1) / DR);
    if constexpr (FA == UT_FMT_INT4 && M >= UT_DOWN_MFMA_MIN_M && M <= 4) {
        if (down_mfma_ok(FA, M, a.I, a.ks)) {
            constexpr int WR = 64 * down_mfma_tw<M>();
            const int gxm = (int)((a.H + WR - 1) / WR);
            if (!b) {
                hipLaunchKernelGGL((k_moe_down_mfma<M>), dim3((unsigned)gxm, (unsigned)slots),
                                   dim3(kGemvThreads), 0, ctx->stream, a);
                return;
            }
            // a shared MLP beside it (one slot, no split): its tiles in the same grid
            constexpr int DRB = 16 * down_rows<M>();
            const int nrouted = gxm * (int)slots;
            const unsigned n = (unsigned)(nrouted + (b->H + DRB - 1) / DRB);
            if (fb == UT_FMT_INT4)
                hipLaunchKernelGGL((k_moe_down_mfma_dual<M, UT_FMT_INT4>), dim3(n), dim3(kGemvThreads), 0,
                                   ctx->stream, a, *b, gxm, nrouted);
            else
                hipLaunchKernelGGL((k_moe_down_mfma_dual<M, UT_FMT_INT8>), dim3(n), dim3(kGemvThreads), 0,
                                   ctx->stream, a, *b, gxm, nrouted);
            return;
        }
    }
    if constexpr (FA == UT_FMT_INT8 && M >= 2 && M <= 4) {
        if (!b && down_i8_mfma_ok(FA, M, a.I, a.ks, a.kslice)) {
            hipLaunchKernelGGL((k_moe_down_i8_mfma<M>),
                               dim3((unsigned)((a.H + 63) / 64), (unsigned)slots, (unsigned)a.ks),
                               dim3(kGemvThreads), 0, ctx->stream, a);
            if (a.ks > 1)
                hipLaunchKernelGGL((k_moe_down_finish<FA>),
                                   dim3((unsigned)((a.H + kGemvThreads - 1) / kGemvThreads),
                                        (unsigned)(slots * M)),
                                   dim3(kGemvThreads), 0, ctx->stream, a, M);
            return;
        }
    }
    if (!b) {
        hipLaunchKernelGGL((k_moe_down<FA, M>), dim3(gx, (unsigned)slots, (unsigned)a.ks),
                           dim3(kGemvThreads), 0, ctx->stream, a);
        if (a.ks > 1)
            hipLaunchKernelGGL((k_moe_down_finish<FA>),
                               dim3((unsigned)((a.H + kGemvThreads - 1) / kGemvThreads),
                                    (unsigned)(slots * M)),
                               dim3(kGemvThreads), 0, ctx->stream, a, M);
        return;
    }
    if constexpr (FA != UT_FMT_F32) {
        const dim3 grid(gx, (unsigned)(slots + 1));
        if (fb == UT_FMT_INT4)
            hipLaunchKernelGGL((k_moe_down_dual<FA, UT_FMT_INT4, M>), grid, dim3(kGemvThreads), 0, ctx->stream, a, *b);
        else
            hipLaunchKernelGGL((k_moe_down_dual<FA, UT_FMT_INT8, M>), grid, dim3(kGemvThreads), 0, ctx->stream, a, *b);
    }
}

template <int FMT, int M>
static int32_t moe_pass_t(ut_ctx *ctx, const MoeCall &c, const ScratchLayout &L, char *base,
                          int64_t slots) {
    MoePlan plan = c.plan ? *c.plan : moe_plan_view(base, L);
    const bool need_plan = !c.plan_ready && !c.plan;
    int tok = -1;
    XSrc xs{};
    const int32_t *xexps = nullptr;
    // expert ids given: the gate/up workgroups resolve the plan themselves
    // (gate_plan); with x not digitised, one row and x staged whole, they
    // digitise x too (self_plan, x as f32)
    constexpr int64_t KC = gemv_chunk_cols<FMT, M>();
    // the matrix-core gate/up (int4, 2..4 rows): x as f32 with the
    // digitiser's exponents, the slot plan made before the launch, a shared
    // expert in the same launches (config-4 verify of two rows: 1,027 ->
    // 1,003 us of GPU time against the dot-product dual kernels); the int8
    // kernel reads x's digit planes only, so caller digits serve it as they
    // are (a model's dense FFN at 2..4 rows)
    const bool use_mfma = gate_up_mfma_ok(FMT, M, c.H) && c.extra_slot < 0 &&
                          (FMT == UT_FMT_INT8 || !c.x_digits || c.x_matches_digits) &&
                          L.ntiles == (c.I + kGateUpRowsPerWG - 1) / kGateUpRowsPerWG;
    const bool gate_plan = FMT != UT_FMT_F32 && need_plan && c.extra_slot < 0 &&
                           (int64_t)M * c.k <= 64 && !use_mfma;
    const bool self_plan = gate_plan && !c.x_digits && !c.shared && c.H <= KC &&
                           c.H % FmtTraits<FMT>::kStepCols == 0 && M == 1;
    const bool gate_plans_here = gate_plan && (self_plan || c.x_digits);
    // routing inside gate/up: one row (at two rows the routing's registers
    // and latency in the prologue cost the expert launch more than the
    // route launch it saves), the wave router with four keys per lane
    int kpl = 0;
    const bool route_here = c.route_logits && gate_plans_here && M == 1 &&
                            route_wave_ok(c.E, c.route_ng, c.route_tg, c.k, &kpl) && kpl == 4;
    if (c.route_logits && !route_here)
        UT_TRY(launch_route(ctx, c.route_logits, c.route_bias, M, c.E, c.k, c.route_ng, c.route_tg,
                            c.route_norm, c.route_scale, c.route_ids, c.route_w));
    // bf16 activations: staged and widened by the gate/up launch itself
    // when it digitises x (self_plan), else widened into the scratch first
    const float *xin = c.x;
    if (c.xh && !(self_plan && FMT != UT_FMT_F32)) {
        float *xw = (float *)(base + L.xw);
        UT_TRY(launch_bf16_to_f32(ctx, c.xh, (int64_t)M * c.H, xw));
        xin = xw;
    }
    if constexpr (FMT == UT_FMT_F32) {
        xs.xf = xin;
        xs.ldx = c.H;
    } else if (self_plan) {
        xs.xf = c.xh ? nullptr : xin;
        xs.xh = c.xh;
        xs.ldx = c.H;
        xs.self_max = 1;
    } else {
        XDigits xd = xdigits_view(base + L.xd, M, c.H, L.xflags);
        if (c.x_digits) {
            xd = *c.x_digits;  // caller already digitised x
        } else if (need_plan && c.extra_slot < 0) {
            UT_TRY(launch_digitize_plan(ctx, xin, M, c.H, xd, L.xflags, c.ids, c.k, c.E,
                                        (const void *const *)c.tbl.gate_w, plan, c.err_flag));
        } else {
            UT_TRY(launch_digitize(ctx, xin, c.H, M, c.H, nullptr, xd, L.xflags));
        }
        xs.dig = FMT == UT_FMT_INT4 ? xd.dig4 : xd.dig8;
        xs.KW = (c.H + FmtTraits<FMT>::kColsPerWord - 1) / FmtTraits<FMT>::kColsPerWord;
        xexps = xd.exps;
    }
    // the gate/up launch (gate_plan) or the digitiser writes the plan
    const bool planned =
        gate_plan || (FMT != UT_FMT_F32 && !c.x_digits && need_plan && c.extra_slot < 0);
    if (need_plan && !planned) {
        tok = timing_begin(ctx, "moe_plan");
        hipLaunchKernelGGL(k_moe_plan, dim3(1), dim3(256), 0, ctx->stream, c.ids, M, c.k, (int)c.E,
                           (const void *const *)c.tbl.gate_w, c.extra_slot, plan, c.err_flag);
        timing_end(ctx, tok);
        UT_TRY(launch_check(ctx, "k_moe_plan"));
    }
    float *h = (float *)(base + L.h);
    uint32_t *hmax = (uint32_t *)(base + L.hmax);
    // the shared MLP's buffers (c.shared)
    ScratchLayout SL;
    char *sbase = (char *)c.shared_scratch;
    if (c.shared) SL = moe_layout(M, 1, 1, c.H, c.shared->I, c.shared->fmt);
    GateUpArgs gb{};
    DownArgs db{};
    float *dshared = nullptr;
    // the combine folded into the down launch (CombineFold): plain combine
    // (no fused norm), the routed experts alone, no K split, rows as
    // k_moe_combine4 takes them
    const bool split_down = slots == 1 && !c.shared;
    const bool fold = UT_MOE_FOLD_COMBINE && !c.next && !c.shared && !split_down && c.H % 4 == 0 &&
                      c.ldo % 4 == 0 && ((uintptr_t)c.out & 15) == 0 &&
                      (!c.init || ((uintptr_t)c.init & 15) == 0);
    int32_t *arrive = fold ? (int32_t *)(base + L.arrive) : nullptr;
    {
        GateUpArgs a;
        a.tbl = c.tbl;
        a.sp = plan.sp;
        a.uniq = plan.uniq;
        a.count = plan.count;
        a.H = c.H;
        a.I = c.I;
        a.row_bytes = payload_bytes(FMT, 1, c.H);
        a.x = xs;
        a.exps = xexps;
        // x digitised in this pass from c.x (so c.x is what the digits
        // hold): the matrix-core kernel stages c.x itself
        if (use_mfma && xs.dig && xexps) {
            if (FMT == UT_FMT_INT4) a.mfma_xf = xin;
            else a.mfma8 = true;
        }
        a.h = h;
        a.hmax_parts = hmax;
        a.ntiles = (int)L.ntiles;
        if (gate_plans_here) {
            a.plan_ids = c.ids;
            a.plan_M = M;
            a.plan_k = c.k;
            a.E = c.E;
            a.ptbl = (const void *const *)c.tbl.gate_w;
            a.plan = plan;
            a.err_flag = c.err_flag;
        }
        if (gate_plans_here && route_here) {
            a.route_lg = c.route_logits;
            a.route_bias = c.route_bias;
            a.route_ng = c.route_ng;
            a.route_tg = c.route_tg;
            a.route_norm = c.route_norm;
            a.route_scale = c.route_scale;
            a.route_ids = c.route_ids;
            a.route_w = c.route_w;
        }
        a.arrive = arrive;
        a.narrive = (int)((c.H + 31) / 32);
        if (c.shared) {
            const MoeCall &sc = *c.shared;
            gb.tbl = sc.tbl;
            gb.sp = sc.plan->sp;
            gb.uniq = sc.plan->uniq;
            gb.count = sc.plan->count;
            gb.H = c.H;
            gb.I = sc.I;
            gb.row_bytes = payload_bytes(sc.fmt, 1, c.H);
            gb.x.dig = sc.fmt == UT_FMT_INT4 ? c.x_digits->dig4 : c.x_digits->dig8;
            gb.x.KW = sc.fmt == UT_FMT_INT4 ? (c.H + 7) / 8 : (c.H + 3) / 4;
            gb.exps = c.x_digits->exps;
            gb.h = (float *)(sbase + SL.h);
            gb.hmax_parts = (uint32_t *)(sbase + SL.hmax);
            gb.ntiles = (int)SL.ntiles;
        }
        tok = timing_begin(ctx, FMT == UT_FMT_INT4 ? "moe_gate_up_int4" : FMT == UT_FMT_INT8 ? "moe_gate_up_int8" : "moe_gate_up_f32");
        launch_gate_up<FMT, M>(ctx, a, slots, c.shared ? &gb : nullptr, c.shared ? c.shared->fmt : 0);
        timing_end(ctx, tok);
        UT_TRY(launch_check(ctx, "k_moe_gate_up"));
    }
    XSrc hs{};
    hs.xf = h;
    hs.ldx = c.I;
    const int64_t hstride = (int64_t)M * c.I;
    float *d = (float *)(base + L.d);
    {
        DownArgs a;
        a.tbl = c.tbl;
        a.sp = plan.sp;
        a.uniq = plan.uniq;
        a.count = plan.count;
        a.H = c.H;
        a.I = c.I;
        a.row_bytes = payload_bytes(FMT, 1, c.I);
        a.x = hs;
        a.x_slot_stride = hstride;
        a.hmax_parts = hmax;
        a.nparts = (int)L.ntiles;
        a.d = d;
        if (fold) {
            a.fold.arrive = arrive;
            a.fold.choice_slot = plan.choice_slot;
            a.fold.weights = c.weights;
            a.fold.k = c.k;
            a.fold.extra = c.extra_slot >= 0 ? 1 : 0;
            a.fold.accumulate = c.accumulate;
            a.fold.init = c.init;
            a.fold.out = c.out;
            a.fold.ldo = c.ldo;
        }
        // a one-slot MLP (dense FFN, lone shared expert) has too few down
        // tiles to fill the chip: split its K range (M-independent choice)
        if (split_down) {
            constexpr int64_t step = FmtTraits<FMT>::kStepCols;
            const int64_t tiles64 = (c.H + 63) / 64;
            int64_t ks = tiles64 >= 256 ? 1 : (512 + tiles64 - 1) / tiles64;
            // integer formats (exact partial totals, so any split gives the
            // same result): slices short enough to stage once
            constexpr int64_t kcd = down_kc<FMT, M>();
            if (FMT != UT_FMT_F32 && ks > 1 && (c.I + ks - 1) / ks > kcd) ks = (c.I + kcd - 1) / kcd;
            if (ks > kDownMaxSplit) ks = kDownMaxSplit;
            if (ks > c.I / (2 * step)) ks = c.I / (2 * step);
            if (ks > 1) {
                int64_t kslice = (c.I + ks - 1) / ks;
                kslice = (kslice + step - 1) / step * step;
                a.ks = (int)((c.I + kslice - 1) / kslice);
                a.kslice = kslice;
                a.part = (int64_t *)(base + L.dpart);
            }
        }
        if (c.shared) {
            const MoeCall &sc = *c.shared;
            db.tbl = sc.tbl;
            db.sp = sc.plan->sp;
            db.uniq = sc.plan->uniq;
            db.count = sc.plan->count;
            db.H = c.H;
            db.I = sc.I;
            db.row_bytes = payload_bytes(sc.fmt, 1, sc.I);
            db.x = XSrc{};
            db.x.xf = gb.h;
            db.x.ldx = sc.I;
            db.x_slot_stride = (int64_t)M * sc.I;
            db.hmax_parts = gb.hmax_parts;
            db.nparts = gb.ntiles;
            db.d = dshared = (float *)(sbase + SL.d);
        }
        tok = timing_begin(ctx, FMT == UT_FMT_INT4 ? "moe_down_int4" : FMT == UT_FMT_INT8 ? "moe_down_int8" : "moe_down_f32");
        launch_down<FMT, M>(ctx, a, slots, c.shared ? &db : nullptr, c.shared ? c.shared->fmt : 0);
        timing_end(ctx, tok);
        UT_TRY(launch_check(ctx, "k_moe_down"));
    }
    if (fold) return UT_OK;
    if (c.next) {
        if (!moe_combine_norm_ok(c.H) || ((uintptr_t)c.out & 15) != 0 || c.ldo % 4 != 0 ||
            (c.init && ((uintptr_t)c.init & 15) != 0) || !c.next->norm_w || !c.next->nd.exps) {
            set_error(ctx, "moe_pass: fused next norm needs H %% 8 == 0, H <= 8192 and 16-byte "
                           "aligned rows (H=%lld)", (long long)c.H);
            return UT_ERR_ARG;
        }
        const NormNext &nx = *c.next;
        RowDigArgs nd{};
        nd.K = c.H;
        nd.norm_w = nx.norm_w;
        nd.eps = nx.eps;
        nd.out = nx.normed;
        nd.ldo = nx.ldn;
        nd.exps = nx.nd.exps;
        nd.dig4 = (nx.flags & XD_DIG4) ? nx.nd.dig4 : nullptr;
        nd.dig8 = (nx.flags & XD_DIG8) ? nx.nd.dig8 : nullptr;
        nd.xt = (nx.flags & XD_XT) ? nx.nd.xt : nullptr;
        nd.raw = c.out;
        nd.raw2 = nx.raw2;
        nd.ldr2 = nx.ld2;
        nd.pos2 = nx.pos2;
        nd.ldr = c.ldo;
        tok = timing_begin(ctx, "moe_combine_norm");
        const unsigned threads = (unsigned)((c.H / 8 + 63) / 64 * 64);
        hipLaunchKernelGGL(k_moe_combine_norm, dim3((unsigned)M), dim3(threads), 0, ctx->stream,
                           plan.choice_slot, c.weights, d, M, c.k, c.H, plan.count,
                           c.extra_slot >= 0 ? 1 : 0, dshared, c.init, c.out, c.ldo, c.accumulate,
                           nd);
        timing_end(ctx, tok);
        return launch_check(ctx, "k_moe_combine_norm");
    }
    tok = timing_begin(ctx, "moe_combine");
    if (c.H % 4 == 0 && c.ldo % 4 == 0 && ((uintptr_t)c.out & 15) == 0 &&
        (!c.init || ((uintptr_t)c.init & 15) == 0))
        hipLaunchKernelGGL(k_moe_combine4, dim3((unsigned)((c.H / 4 + 255) / 256), (unsigned)M),
                           dim3(256), 0, ctx->stream, plan.choice_slot, c.weights, d, M, c.k, c.H,
                           plan.count, c.extra_slot >= 0 ? 1 : 0, dshared, c.init, c.out, c.ldo,
                           c.accumulate);
    else
        hipLaunchKernelGGL(k_moe_combine, dim3((unsigned)((c.H + 255) / 256), (unsigned)M),
                           dim3(256), 0, ctx->stream, plan.choice_slot, c.weights, d, M, c.k, c.H,
                           plan.count, c.extra_slot >= 0 ? 1 : 0, dshared, c.init, c.out, c.ldo,
                           c.accumulate);
    timing_end(ctx, tok);
    return launch_check(ctx, "k_moe_combine");
}

template <int FMT>
static int32_t moe_pass_fmt(ut_ctx *ctx, const MoeCall &c, const ScratchLayout &L, char *base,
                            int64_t slots) {
    switch (c.M) {
    case 1: return moe_pass_t<FMT, 1>(ctx, c, L, base, slots);
    case 2: return moe_pass_t<FMT, 2>(ctx, c, L, base, slots);
    case 3: return moe_pass_t<FMT, 3>(ctx, c, L, base, slots);
    default: return moe_pass_t<FMT, 4>(ctx, c, L, base, slots);
    }
}

MoePlan moe_plan_view(void *scratch, const ScratchLayout &L) {
    char *base = (char *)scratch;
    MoePlan plan;
    plan.count = (int32_t *)(base + L.count);
    plan.uniq = (int32_t *)(base + L.uniq);
    plan.choice_slot = (int32_t *)(base + L.choice);
    plan.sp = (const void **)(base + L.sp);
    return plan;
}

bool moe_shape_ok(int fmt, int64_t H, int64_t I) {
    if (fmt == UT_FMT_INT4) return H % 32 == 0 && I % 32 == 0;
    if (fmt == UT_FMT_INT8) return H % 16 == 0 && I % 16 == 0;
    return H % 4 == 0 && I % 4 == 0;
}

int32_t moe_pass(ut_ctx *ctx, const MoeCall &c, void *scratch) {
    if (c.M < 1 || c.M > 4) {
        set_error(ctx, "moe_pass: M=%d outside 1..4", c.M);
        return UT_ERR_ARG;
    }
    if (c.shared) {
        const MoeCall &sc = *c.shared;
        const int need = (sc.fmt == UT_FMT_INT4 ? XD_DIG4 : XD_DIG8) |
                         (c.fmt == UT_FMT_INT4 ? XD_DIG4 : XD_DIG8);
        const bool have = c.x_digits && (!(need & XD_DIG4) || c.x_digits->dig4) &&
                          (!(need & XD_DIG8) || c.x_digits->dig8);
        if (!moe_dual_ok(c.fmt, sc.fmt) || !sc.plan || !c.shared_scratch || !have ||
            !moe_shape_ok(sc.fmt, c.H, sc.I) || c.extra_slot >= 0) {
            set_error(ctx, "moe_pass: shared MLP (format %d) cannot run beside format %d experts",
                      sc.fmt, c.fmt);
            return UT_ERR_ARG;
        }
    }
    if (!moe_shape_ok(c.fmt, c.H, c.I)) {
        set_error(ctx, "moe: hidden %lld / inter %lld not supported for format %d", (long long)c.H,
                  (long long)c.I, c.fmt);
        return UT_ERR_SHAPE;
    }
    const int64_t slots = moe_slots(c.M, c.k, c.E, c.extra_slot);
    ScratchLayout L = moe_layout(c.M, c.k, slots, c.H, c.I, c.fmt);
    char *base = (char *)scratch;
    if (c.fmt == UT_FMT_INT4) return moe_pass_fmt<UT_FMT_INT4>(ctx, c, L, base, slots);
    if (c.fmt == UT_FMT_INT8) return moe_pass_fmt<UT_FMT_INT8>(ctx, c, L, base, slots);
    return moe_pass_fmt<UT_FMT_F32>(ctx, c, L, base, slots);
}

}  // namespace ut

using namespace ut;

struct ut_expert_table {
    ut_ctx *ctx = nullptr;
    int64_t n = 0, hidden = 0, inter = 0;
    int32_t fmt = -1;
    std::vector<const ut_qtensor *> gate, up, down;
    // device arrays: gate_w, up_w, down_w (uint8_t*), gate_s, up_s, down_s (float*)
    void *dev = nullptr;
    ExpertPtrs ptrs{};
    int device = 0;
};

extern "C" {

int32_t ut_route(ut_ctx *ctx, const float *logits_dev, const float *bias_dev, int64_t rows,
                 int64_t n_experts, int32_t top_k, int32_t n_group, int32_t topk_group,
                 int32_t norm_topk_prob, float routed_scaling_factor, int32_t *ids_dev,
                 float *weights_dev) {
    if (!ctx || !logits_dev || !ids_dev || !weights_dev || rows < 0 || n_experts <= 0 ||
        top_k <= 0 || top_k > 64 || n_group < 0 || n_group > 64 || topk_group < 0) {
        set_error(ctx, "ut_route: bad argument (top_k must be 1..64, n_group <= 64)");
        return UT_ERR_ARG;
    }
    if (n_experts > 4096) {
        set_error(ctx, "ut_route: n_experts %lld > 4096", (long long)n_experts);
        return UT_ERR_ARG;
    }
    return launch_route(ctx, logits_dev, bias_dev, rows, n_experts, top_k, n_group, topk_group,
                        norm_topk_prob, routed_scaling_factor, ids_dev, weights_dev);
}

int32_t ut_expert_table_create(ut_ctx *ctx, int64_t n_experts, int64_t hidden, int64_t inter,
                               ut_expert_table **out) {
    if (!ctx || !out || n_experts <= 0 || hidden <= 0 || inter <= 0) return UT_ERR_ARG;
    *out = nullptr;
    ut_expert_table *t = new (std::nothrow) ut_expert_table();
    if (!t) return UT_ERR_OOM;
    t->ctx = ctx;
    t->n = n_experts;
    t->hidden = hidden;
    t->inter = inter;
    t->device = ctx->device;
    t->gate.assign(n_experts, nullptr);
    t->up.assign(n_experts, nullptr);
    t->down.assign(n_experts, nullptr);
    size_t bytes = (size_t)n_experts * sizeof(void *) * 6;
    if (hipMalloc(&t->dev, bytes) != hipSuccess) {
        (void)hipGetLastError();
        delete t;
        return UT_ERR_OOM;
    }
    if (hipMemset(t->dev, 0, bytes) != hipSuccess) {
        (void)hipFree(t->dev);
        delete t;
        return UT_ERR_HIP;
    }
    void **p = (void **)t->dev;
    t->ptrs.gate_w = (const uint8_t *const *)(p);
    t->ptrs.up_w = (const uint8_t *const *)(p + n_experts);
    t->ptrs.down_w = (const uint8_t *const *)(p + 2 * n_experts);
    t->ptrs.gate_s = (const float *const *)(p + 3 * n_experts);
    t->ptrs.up_s = (const float *const *)(p + 4 * n_experts);
    t->ptrs.down_s = (const float *const *)(p + 5 * n_experts);
    *out = t;
    return UT_OK;
}

int32_t ut_expert_table_set(ut_expert_table *t, int64_t e, const ut_qtensor *gate,
                            const ut_qtensor *up, const ut_qtensor *down) {
    if (!t || !gate || !up || !down) return UT_ERR_ARG;
    ut_ctx *ctx = t->ctx;
    if (e < 0 || e >= t->n) {
        set_error(ctx, "expert %lld out of range %lld", (long long)e, (long long)t->n);
        return UT_ERR_BAD_EXPERT;
    }
    if (gate->out_dim != t->inter || gate->in_dim != t->hidden || up->out_dim != t->inter ||
        up->in_dim != t->hidden || down->out_dim != t->hidden || down->in_dim != t->inter) {
        set_error(ctx, "expert %lld: shapes do not match [%lld,%lld]/[%lld,%lld]", (long long)e,
                  (long long)t->inter, (long long)t->hidden, (long long)t->hidden,
                  (long long)t->inter);
        return UT_ERR_SHAPE;
    }
    if (gate->fmt != up->fmt || gate->fmt != down->fmt || (t->fmt >= 0 && gate->fmt != t->fmt)) {
        set_error(ctx, "expert %lld: all experts of a table must share one format", (long long)e);
        return UT_ERR_FORMAT;
    }
    t->fmt = gate->fmt;
    t->gate[e] = gate;
    t->up[e] = up;
    t->down[e] = down;
    void *vals[6] = {gate->payload, up->payload, down->payload, gate->scales, up->scales,
                     down->scales};
    void **p = (void **)t->dev;
    for (int i = 0; i < 6; i++)
        UT_CHECK_HIP(ctx, hipMemcpy(p + i * t->n + e, &vals[i], sizeof(void *), hipMemcpyHostToDevice));
    return UT_OK;
}

void ut_expert_table_free(ut_expert_table *t) {
    if (!t) return;
    (void)hipSetDevice(t->device);
    if (t->dev) (void)hipFree(t->dev);
    delete t;
}

}  // extern "C"

namespace {

// The routed-expert block over rows already routed, in passes of up to four
// rows, with `scratch` (moe_layout's bytes at four rows) as working memory.
int32_t moe_experts_rows(ut_ctx *ctx, const ut_expert_table *tbl, const int32_t *ids_dev,
                         const float *weights_dev, int64_t rows, int32_t top_k, const float *x_dev,
                         float *out_dev, void *scratch, int32_t *flag,
                         const uint16_t *xh_dev = nullptr) {
    const int64_t maxM = 4;
    for (int64_t s0 = 0; s0 < rows; s0 += maxM) {
        MoeCall c;
        c.fmt = tbl->fmt;
        c.tbl = tbl->ptrs;
        c.E = tbl->n;
        c.H = tbl->hidden;
        c.I = tbl->inter;
        c.M = (int)((rows - s0) < maxM ? (rows - s0) : maxM);
        c.k = top_k;
        c.ids = ids_dev + s0 * top_k;
        c.weights = weights_dev + s0 * top_k;
        if (xh_dev)
            c.xh = xh_dev + s0 * tbl->hidden;
        else
            c.x = x_dev + s0 * tbl->hidden;
        c.out = out_dev + s0 * tbl->hidden;
        c.ldo = tbl->hidden;
        c.err_flag = flag;
        UT_TRY(moe_pass(ctx, c, scratch));
    }
    return UT_OK;
}

// bf16 activations are read 8 bytes (four values) at a time: 16-byte
// aligned rows of a hidden size that is a multiple of 8.
bool bf16_rows_ok(ut_ctx *ctx, const char *fn, const uint16_t *x, int64_t hidden) {
    if (((uintptr_t)x & 15) || (hidden & 7)) {
        set_error(ctx, "%s: bf16 activations need 16-byte alignment and hidden %% 8 == 0", fn);
        return false;
    }
    return true;
}

int32_t moe_experts_check(ut_ctx *ctx, const char *fn, const ut_expert_table *tbl,
                          const int32_t *ids_dev, const float *weights_dev, int64_t rows,
                          int32_t top_k, const float *x_dev, float *out_dev) {
    if (!ctx || !tbl || !ids_dev || !weights_dev || !x_dev || !out_dev || rows < 0 || top_k <= 0 ||
        top_k > 64) {
        set_error(ctx, "%s: bad argument", fn);
        return UT_ERR_ARG;
    }
    if (tbl->fmt < 0) {
        set_error(ctx, "%s: empty expert table", fn);
        return UT_ERR_BAD_EXPERT;
    }
    return UT_OK;
}

}  // namespace

// Working memory of ut_moe_experts_noalloc: a fixed array in the code
// object, one copy per device (each GPU the library runs on holds it until
// the process ends).  Host code never names it: kernels get the address
// that hipGetSymbolAddress returned for the device (ctx->noalloc_scratch).
constexpr size_t kNoAllocScratchBytes = size_t(32) << 20;
static __device__ __align__(256) unsigned char noalloc_scratch[kNoAllocScratchBytes];

// The context that owns each device's array: the first to call
// ut_moe_experts_noalloc on that device, until it is destroyed.  Calls from
// any other context on the device are refused (UT_ERR_STATE) instead of
// racing on the array; one context orders its calls on its stream.
namespace {
constexpr int kNoAllocMaxDevices = 64;
std::mutex g_noalloc_mu;
const ut_ctx *g_noalloc_owner[kNoAllocMaxDevices] = {};

int32_t noalloc_claim(ut_ctx *ctx) {
    if (ctx->device < 0 || ctx->device >= kNoAllocMaxDevices) return UT_ERR_ARG;
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    const ut_ctx *&o = g_noalloc_owner[ctx->device];
    if (!o) o = ctx;
    if (o != ctx) {
        set_error(ctx, "ut_moe_experts_noalloc: device %d's working array belongs to another "
                       "context; calls from two contexts would race on it",
                  ctx->device);
        return UT_ERR_STATE;
    }
    return UT_OK;
}
}  // namespace

void ut::moe_noalloc_release(const ut_ctx *ctx) {
    if (ctx->device < 0 || ctx->device >= kNoAllocMaxDevices) return;
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    if (g_noalloc_owner[ctx->device] == ctx) g_noalloc_owner[ctx->device] = nullptr;
}

int32_t ut::moe_noalloc_scratch_init(ut_ctx *ctx) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(noalloc_scratch));
    if (e != hipSuccess || !p) {
        (void)hipGetLastError();
        set_error(ctx, "hipGetSymbolAddress of the expert block's working array failed: %s",
                  hipGetErrorString(e));
        return UT_ERR_HIP;
    }
    ctx->noalloc_scratch = p;
    return UT_OK;
}

extern "C" {

int32_t ut_moe_experts(ut_ctx *ctx, const ut_expert_table *tbl, const int32_t *ids_dev,
                       const float *weights_dev, int64_t rows, int32_t top_k, const float *x_dev,
                       float *out_dev) {
    UT_TRY(moe_experts_check(ctx, "ut_moe_experts", tbl, ids_dev, weights_dev, rows, top_k, x_dev,
                             out_dev));
    if (rows == 0) return UT_OK;
    const int64_t maxM = 4;
    const int64_t slots = moe_slots((int)maxM, top_k, tbl->n, -1);
    ScratchPlan plan;
    plan.add(moe_layout(maxM, top_k, slots, tbl->hidden, tbl->inter, tbl->fmt).total);
    std::vector<void *> ptrs;
    UT_TRY(scratch_acquire(ctx, plan, ptrs));
    int32_t *flag = nullptr;
    UT_TRY(device_error_flag(ctx, &flag));
    return moe_experts_rows(ctx, tbl, ids_dev, weights_dev, rows, top_k, x_dev, out_dev, ptrs[0],
                            flag);
}

int32_t ut_moe_experts_noalloc(ut_ctx *ctx, const ut_expert_table *tbl, const int32_t *ids_dev,
                               const float *weights_dev, int64_t rows, int32_t top_k,
                               const float *x_dev, float *out_dev) {
    // ut_moe_experts without any allocation: the same kernels over the
    // device's fixed working array.  Every byte a pass reads from it was
    // written earlier in the same pass (slot plan, h and its partial maxima,
    // digits, down outputs), so nothing needs clearing between calls.
    UT_TRY(moe_experts_check(ctx, "ut_moe_experts_noalloc", tbl, ids_dev, weights_dev, rows,
                             top_k, x_dev, out_dev));
    if (!ctx->noalloc_scratch || !ctx->dev_err) {
        set_error(ctx, "ut_moe_experts_noalloc: context set-up incomplete");
        return UT_ERR_STATE;
    }
    const int64_t maxM = 4;
    const int64_t slots = moe_slots((int)maxM, top_k, tbl->n, -1);
    const size_t need = moe_layout(maxM, top_k, slots, tbl->hidden, tbl->inter, tbl->fmt).total;
    if (need > kNoAllocScratchBytes) {
        set_error(ctx,
                  "ut_moe_experts_noalloc: working set of %zu bytes (top_k %d, hidden %lld, "
                  "inter %lld) exceeds the fixed %zu-byte array; use ut_moe_experts",
                  need, top_k, (long long)tbl->hidden, (long long)tbl->inter,
                  kNoAllocScratchBytes);
        return UT_ERR_ARG;
    }
    UT_TRY(noalloc_claim(ctx));
    if (rows == 0) return UT_OK;
    return moe_experts_rows(ctx, tbl, ids_dev, weights_dev, rows, top_k, x_dev, out_dev,
                            ctx->noalloc_scratch, ctx->dev_err);
}

}  // extern "C"

namespace {

// ut_moe_route_experts over f32 (x_dev) or bf16 (xh_dev) activations.
int32_t moe_route_experts_any(ut_ctx *ctx, const char *fn, const ut_expert_table *tbl,
                              const float *logits_dev, const float *bias_dev, int64_t rows,
                              int32_t top_k, int32_t n_group, int32_t topk_group,
                              int32_t norm_topk_prob, float routed_scaling_factor,
                              const float *x_dev, const uint16_t *xh_dev, float *out_dev,
                              int32_t *ids_dev, float *weights_dev) {
    if (!ctx || !tbl || !logits_dev || !ids_dev || !weights_dev || !(x_dev || xh_dev) ||
        !out_dev || rows < 0 || top_k <= 0 || top_k > 64 || n_group < 0 || n_group > 64 ||
        topk_group < 0) {
        set_error(ctx, "%s: bad argument (top_k must be 1..64, n_group <= 64)", fn);
        return UT_ERR_ARG;
    }
    if (tbl->n > 4096) {
        set_error(ctx, "%s: n_experts %lld > 4096", fn, (long long)tbl->n);
        return UT_ERR_ARG;
    }
    if (tbl->fmt < 0) {
        set_error(ctx, "%s: empty expert table", fn);
        return UT_ERR_BAD_EXPERT;
    }
    if (xh_dev && !bf16_rows_ok(ctx, fn, xh_dev, tbl->hidden)) return UT_ERR_ARG;
    if (rows == 0) return UT_OK;
    const int64_t maxM = 4;
    const int64_t slots = moe_slots((int)maxM, top_k, tbl->n, -1);
    ScratchPlan plan;
    plan.add(moe_layout(maxM, top_k, slots, tbl->hidden, tbl->inter, tbl->fmt).total);
    std::vector<void *> ptrs;
    UT_TRY(scratch_acquire(ctx, plan, ptrs));
    int32_t *flag = nullptr;
    UT_TRY(device_error_flag(ctx, &flag));
    for (int64_t s0 = 0; s0 < rows; s0 += maxM) {
        MoeCall c;
        c.fmt = tbl->fmt;
        c.tbl = tbl->ptrs;
        c.E = tbl->n;
        c.H = tbl->hidden;
        c.I = tbl->inter;
        c.M = (int)((rows - s0) < maxM ? (rows - s0) : maxM);
        c.k = top_k;
        // the choices: routed inside the gate/up launch where that applies
        // (one row, the one-wave router), else by a route launch first
        c.route_logits = logits_dev + s0 * tbl->n;
        c.route_bias = bias_dev;
        c.route_ng = n_group;
        c.route_tg = topk_group;
        c.route_norm = norm_topk_prob;
        c.route_scale = routed_scaling_factor;
        c.route_ids = ids_dev + s0 * top_k;
        c.route_w = weights_dev + s0 * top_k;
        c.ids = c.route_ids;
        c.weights = c.route_w;
        if (xh_dev)
            c.xh = xh_dev + s0 * tbl->hidden;
        else
            c.x = x_dev + s0 * tbl->hidden;
        c.out = out_dev + s0 * tbl->hidden;
        c.ldo = tbl->hidden;
        c.err_flag = flag;
        UT_TRY(moe_pass(ctx, c, ptrs[0]));
    }
    return UT_OK;
}

}  // namespace

extern "C" {

int32_t ut_moe_route_experts(ut_ctx *ctx, const ut_expert_table *tbl, const float *logits_dev,
                             const float *bias_dev, int64_t rows, int32_t top_k, int32_t n_group,
                             int32_t topk_group, int32_t norm_topk_prob,
                             float routed_scaling_factor, const float *x_dev, float *out_dev,
                             int32_t *ids_dev, float *weights_dev) {
    if (!x_dev) {
        set_error(ctx, "ut_moe_route_experts: bad argument");
        return UT_ERR_ARG;
    }
    return moe_route_experts_any(ctx, "ut_moe_route_experts", tbl, logits_dev, bias_dev, rows,
                                 top_k, n_group, topk_group, norm_topk_prob,
                                 routed_scaling_factor, x_dev, nullptr, out_dev, ids_dev,
                                 weights_dev);
}

int32_t ut_moe_route_experts_bf16(ut_ctx *ctx, const ut_expert_table *tbl,
                                  const float *logits_dev, const float *bias_dev, int64_t rows,
                                  int32_t top_k, int32_t n_group, int32_t topk_group,
                                  int32_t norm_topk_prob, float routed_scaling_factor,
                                  const uint16_t *x_dev, float *out_dev, int32_t *ids_dev,
                                  float *weights_dev) {
    if (!x_dev) {
        set_error(ctx, "ut_moe_route_experts_bf16: bad argument");
        return UT_ERR_ARG;
    }
    return moe_route_experts_any(ctx, "ut_moe_route_experts_bf16", tbl, logits_dev, bias_dev,
                                 rows, top_k, n_group, topk_group, norm_topk_prob,
                                 routed_scaling_factor, nullptr, x_dev, out_dev, ids_dev,
                                 weights_dev);
}

int32_t ut_moe_experts_bf16(ut_ctx *ctx, const ut_expert_table *tbl, const int32_t *ids_dev,
                            const float *weights_dev, int64_t rows, int32_t top_k,
                            const uint16_t *x_dev, float *out_dev) {
    const float *fake = (const float *)x_dev;  // the argument check's non-null test only
    UT_TRY(moe_experts_check(ctx, "ut_moe_experts_bf16", tbl, ids_dev, weights_dev, rows, top_k,
                             fake, out_dev));
    if (!bf16_rows_ok(ctx, "ut_moe_experts_bf16", x_dev, tbl->hidden)) return UT_ERR_ARG;
    if (rows == 0) return UT_OK;
    const int64_t maxM = 4;
    const int64_t slots = moe_slots((int)maxM, top_k, tbl->n, -1);
    ScratchPlan plan;
    plan.add(moe_layout(maxM, top_k, slots, tbl->hidden, tbl->inter, tbl->fmt).total);
    std::vector<void *> ptrs;
    UT_TRY(scratch_acquire(ctx, plan, ptrs));
    int32_t *flag = nullptr;
    UT_TRY(device_error_flag(ctx, &flag));
    return moe_experts_rows(ctx, tbl, ids_dev, weights_dev, rows, top_k, nullptr, out_dev, ptrs[0],
                            flag, x_dev);
}

}  // extern "C"
