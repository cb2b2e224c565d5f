// ut_model.hip -- the DeepSeek model, inference session and MTP
// draft+verify loop on one HIP stream (adapters/undertow-deepseek-moe/src/
// {loader,model,attention,mtp}.rs).
//
// All activations, the compressed KV caches and the hidden states kept for
// the MTP head stay in HBM.  Per step the host only sends token ids and
// reads back argmax ids (a few ints) to make the accept decision.
#include <cmath>
#include <cstring>
#include <string>
#include <unordered_map>

#include "ut_mla.h"
#include "ut_moe.h"
#include "ut_ops.h"
#include "ut_safetensors.h"
#include "ut_sample.h"
#include "ut_store.h"

using namespace ut;

namespace {

struct DevTensor {
    ut_qtensor *qt = nullptr;  // matrices
    float *vec = nullptr;      // 1-D f32 vectors
    int64_t d0 = 0, d1 = 0;
};

// One MLP (dense FFN, shared expert) as a one-slot expert table, so the
// fused gate/up + down kernels serve it too.
struct MlpW {
    const ut_qtensor *gate = nullptr, *up = nullptr, *down = nullptr;
    void *dev = nullptr;  // 6 device pointers
    ExpertPtrs ptrs{};
    int fmt = UT_FMT_F32;
    int64_t inter = 0;
};

struct LayerW {
    const float *input_norm = nullptr, *post_norm = nullptr;
    bool lora = false;
    const ut_qtensor *q_a = nullptr, *q_b = nullptr, *q_proj = nullptr, *kv_a = nullptr,
                     *kv_b = nullptr, *o_proj = nullptr;
    const float *q_a_norm = nullptr, *kv_a_norm = nullptr;
    bool dense = false;
    MlpW mlp;                        // dense FFN
    const ut_qtensor *gate = nullptr;  // router [E, H] f32
    const float *bias = nullptr;
    bool has_shared = false;
    MlpW shared;
    void *experts_dev = nullptr;     // 6*E device pointers
    ExpertPtrs experts{};
    std::vector<const ut_qtensor *> eqt;  // [E][3] gate, up, down (resident experts)
    int expert_fmt = UT_FMT_F32;
    int64_t index = 0;               // layer index (the MTP layer: num_hidden_layers)
};

struct KvCache {
    float *latent = nullptr;  // [cap, kv_lora]
    float *krot = nullptr;    // [cap, rope]
    __bf16 *kc = nullptr;     // split bf16 form [cap][2][kv_lora + rope] (MFMA attention)
    int64_t len = 0;
};

}  // namespace

struct ut_model {
    ut_ctx *ctx = nullptr;
    ut_model_config c{};
    std::unordered_map<std::string, DevTensor> tensors;
    std::vector<LayerW> layers;
    LayerW mtp_layer;
    bool has_mtp = false;
    const ut_qtensor *embed = nullptr, *lm_head = nullptr, *eh_proj = nullptr, *mtp_head = nullptr;
    const float *final_norm = nullptr, *enorm = nullptr, *hnorm = nullptr, *mtp_norm = nullptr;
    float2 *rope_table = nullptr;  // [max_pos][rope/2]
    int32_t *zeros = nullptr;      // [4] expert id 0 (MLP as a one-slot table)
    float *ones = nullptr;         // [4] weight 1
    MoePlan mlp_plan{};            // the fixed one-slot plan of an MLP
    bool finalized = false;
    std::vector<int32_t> stop_ids;  // the checkpoint's stop tokens (DeepseekMoeModel::stop_ids)
    ut::ExpertStore *store = nullptr;  // the HBM tier of routed experts, when not all resident
    bool store_prefetch = false;       // pilot-router hints one layer ahead at decode
    bool graphs = false;               // one-row decode steps replayed from a captured graph
    int64_t graph_captures = 0, graph_replays = 0, graph_failures = 0;
    std::vector<void *> device_allocs;
    int64_t device_bytes = 0;
    int device = 0;
    int refs = 1;  // the creator + one per live session
    // a session KV budget in bytes (LoadOptions::kv_budget_bytes), -1: none;
    // it lowers the positions a session may hold (ut_model_max_context)
    int64_t kv_budget = -1;
};

namespace {

struct Workspace {
    int64_t rows = 0;
    void *base = nullptr;
    size_t bytes = 0;
    float *x = nullptr, *normed = nullptr, *attn = nullptr, *moe_out = nullptr;
    float *qa = nullptr, *qa_n = nullptr, *q = nullptr, *comp = nullptr;
    float *qabs = nullptr, *qrope = nullptr, *clat = nullptr, *ctxv = nullptr;
    float *logits = nullptr, *emb = nullptr, *cat = nullptr;
    float *rlogits = nullptr, *rw = nullptr;
    int32_t *rids = nullptr, *ids = nullptr, *am = nullptr, *err = nullptr;
    int32_t *vids = nullptr;  // verify ids [next, drafts...] assembled on the device
    uint32_t *vmax = nullptr;  // partial maxima of |ctx| per row (absorb_v -> o_proj)
    int32_t *vexps = nullptr;  // o_proj activation exponents per row
    void *digits = nullptr, *moe = nullptr, *mla = nullptr, *argm = nullptr;
    void *digA = nullptr, *digB = nullptr;  // activation digits shared by consumers
    float *fast = nullptr;  // the fast-int8 path's MLP rows
};

}  // namespace

struct ut_session {
    ut_model *m = nullptr;
    // the context (stream, scratch, pinned staging) the session's work runs
    // on: the model's, or one of the caller's on the same device
    ut_ctx *ctx = nullptr;
    int32_t path = 0;
    int64_t pos = 0;
    std::vector<KvCache> kv;
    KvCache mtp_kv;
    int64_t mtp_fed = 0;
    std::vector<int32_t> tokens;
    float *hidden = nullptr;  // [cap, H] pre-final-norm hidden states (MTP input)
    void *kv_alloc = nullptr;
    Workspace ws;
    int64_t cap = 0;
    // host staging of the generation loops (pinned): [0, kPinIds) ids going
    // up, then readback slots; `ready` marks the end of the last readback
    int32_t *pin = nullptr;
    hipEvent_t ready = nullptr;
    // where the last readback put the sticky error flag (an int of the
    // readback slot: its last one, or just after the argmax rows)
    int64_t err_slot = 63;
    // The one-row decode step as a captured graph (ut_model_enable_graphs):
    // the device word holding the step's position, the position it will hold
    // once the enqueued work has run (-1: unknown), the executable graph, the
    // one-row steps run so far, and whether capturing failed (eager from
    // then on).
    int64_t *dpos = nullptr;
    int64_t dpos_host = -1;
    hipGraphExec_t g1 = nullptr;
    int64_t m1_steps = 0;
    // the MTP verify step (gv_rows rows fed from ws.vids), captured likewise
    hipGraphExec_t gv = nullptr;
    int64_t gv_rows = 0, v_steps = 0;
    // the MTP head's feed after a verify, one graph per fed row count 1..4
    hipGraphExec_t gd[4] = {nullptr, nullptr, nullptr, nullptr};
    int64_t d_steps[4] = {0, 0, 0, 0};
    bool graph_failed = false;
};

namespace {

constexpr int64_t kMlaRowsPerCall = 16;
constexpr int64_t kPinIds = 16384;   // ints of the upload slot (the last 8: verify ids)
constexpr int64_t kPinBack = 64;     // ints of the readback slot (argmax rows, drafts, flag)

int64_t hd(const ut_model *m) { return m->c.hidden_size; }

uint64_t mix_host(uint64_t seed, uint64_t i) {
    uint64_t z = seed * 0x9e3779b97f4a7c15ull + i + 1;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

int32_t dev_alloc(ut_model *m, size_t bytes, void **p) {
    if (hipMalloc(p, bytes) != hipSuccess) {
        (void)hipGetLastError();
        set_error(m->ctx, "device allocation of %zu bytes failed", bytes);
        return UT_ERR_OOM;
    }
    m->device_allocs.push_back(*p);
    m->device_bytes += (int64_t)bytes;
    return UT_OK;
}

const DevTensor *find(const ut_model *m, const std::string &name) {
    auto it = m->tensors.find(name);
    return it == m->tensors.end() ? nullptr : &it->second;
}

int32_t get_qt(ut_model *m, const std::string &name, int64_t o, int64_t i, const ut_qtensor **out) {
    const DevTensor *t = find(m, name);
    if (!t || !t->qt) {
        set_error(m->ctx, "missing tensor %s", name.c_str());
        return UT_ERR_NOT_FOUND;
    }
    if (t->qt->out_dim != o || t->qt->in_dim != i) {
        set_error(m->ctx, "tensor %s has shape [%lld, %lld], expected [%lld, %lld]", name.c_str(),
                  (long long)t->qt->out_dim, (long long)t->qt->in_dim, (long long)o, (long long)i);
        return UT_ERR_SHAPE;
    }
    *out = t->qt;
    return UT_OK;
}

int32_t get_vec(ut_model *m, const std::string &name, int64_t n, const float **out) {
    const DevTensor *t = find(m, name);
    if (!t || !t->vec) {
        set_error(m->ctx, "missing tensor %s", name.c_str());
        return UT_ERR_NOT_FOUND;
    }
    if (t->d0 * t->d1 != n) {
        set_error(m->ctx, "tensor %s has %lld elements, expected %lld", name.c_str(),
                  (long long)(t->d0 * t->d1), (long long)n);
        return UT_ERR_SHAPE;
    }
    *out = t->vec;
    return UT_OK;
}

int32_t make_mlp(ut_model *m, const std::string &prefix, int64_t inter, MlpW *w) {
    const int64_t H = hd(m);
    UT_TRY(get_qt(m, prefix + "gate_proj.weight", inter, H, &w->gate));
    UT_TRY(get_qt(m, prefix + "up_proj.weight", inter, H, &w->up));
    UT_TRY(get_qt(m, prefix + "down_proj.weight", H, inter, &w->down));
    if (w->gate->fmt != w->up->fmt || w->gate->fmt != w->down->fmt) {
        set_error(m->ctx, "%s: gate/up/down must share one format", prefix.c_str());
        return UT_ERR_FORMAT;
    }
    w->fmt = w->gate->fmt;
    w->inter = inter;
    if (!moe_shape_ok(w->fmt, H, inter)) {
        set_error(m->ctx, "%s: hidden %lld / inter %lld unsupported for format %d", prefix.c_str(),
                  (long long)H, (long long)inter, w->fmt);
        return UT_ERR_SHAPE;
    }
    UT_TRY(dev_alloc(m, 6 * sizeof(void *), &w->dev));
    const void *vals[6] = {w->gate->payload, w->up->payload, w->down->payload, w->gate->scales,
                           w->up->scales, w->down->scales};
    UT_CHECK_HIP(m->ctx, hipMemcpy(w->dev, vals, sizeof vals, hipMemcpyHostToDevice));
    void **p = (void **)w->dev;
    w->ptrs.gate_w = (const uint8_t *const *)(p + 0);
    w->ptrs.up_w = (const uint8_t *const *)(p + 1);
    w->ptrs.down_w = (const uint8_t *const *)(p + 2);
    w->ptrs.gate_s = (const float *const *)(p + 3);
    w->ptrs.up_s = (const float *const *)(p + 4);
    w->ptrs.down_s = (const float *const *)(p + 5);
    return UT_OK;
}

// load_layer (adapters/undertow-deepseek-moe/src/loader.rs:67-174)
int32_t load_layer(ut_model *m, int64_t li, bool dense, LayerW *L) {
    const ut_model_config &c = m->c;
    const int64_t H = c.hidden_size, heads = c.num_attention_heads;
    const int64_t qh = c.qk_nope_head_dim + c.qk_rope_head_dim;
    const std::string p = "model.layers." + std::to_string(li) + ".";
    UT_TRY(get_vec(m, p + "input_layernorm.weight", H, &L->input_norm));
    UT_TRY(get_vec(m, p + "post_attention_layernorm.weight", H, &L->post_norm));
    if (c.q_lora_rank > 0) {
        L->lora = true;
        UT_TRY(get_qt(m, p + "self_attn.q_a_proj.weight", c.q_lora_rank, H, &L->q_a));
        UT_TRY(get_vec(m, p + "self_attn.q_a_layernorm.weight", c.q_lora_rank, &L->q_a_norm));
        UT_TRY(get_qt(m, p + "self_attn.q_b_proj.weight", heads * qh, c.q_lora_rank, &L->q_b));
    } else {
        UT_TRY(get_qt(m, p + "self_attn.q_proj.weight", heads * qh, H, &L->q_proj));
    }
    UT_TRY(get_qt(m, p + "self_attn.kv_a_proj_with_mqa.weight", c.kv_lora_rank + c.qk_rope_head_dim,
                  H, &L->kv_a));
    UT_TRY(get_vec(m, p + "self_attn.kv_a_layernorm.weight", c.kv_lora_rank, &L->kv_a_norm));
    UT_TRY(get_qt(m, p + "self_attn.kv_b_proj.weight", heads * (c.qk_nope_head_dim + c.v_head_dim),
                  c.kv_lora_rank, &L->kv_b));
    UT_TRY(get_qt(m, p + "self_attn.o_proj.weight", H, heads * c.v_head_dim, &L->o_proj));
    L->dense = dense;
    if (dense) {
        UT_TRY(make_mlp(m, p + "mlp.", c.intermediate_size, &L->mlp));
        return UT_OK;
    }
    const int64_t E = c.n_routed_experts;
    UT_TRY(get_qt(m, p + "mlp.gate.weight", E, H, &L->gate));
    if (L->gate->fmt != UT_FMT_F32) {
        set_error(m->ctx, "%smlp.gate.weight must stay f32", p.c_str());
        return UT_ERR_FORMAT;
    }
    if (find(m, p + "mlp.gate.e_score_correction_bias"))
        UT_TRY(get_vec(m, p + "mlp.gate.e_score_correction_bias", E, &L->bias));
    if (c.n_shared_experts > 0) {
        L->has_shared = true;
        UT_TRY(make_mlp(m, p + "mlp.shared_experts.", c.n_shared_experts * c.moe_intermediate_size,
                        &L->shared));
    }
    UT_TRY(dev_alloc(m, (size_t)E * 6 * sizeof(void *), &L->experts_dev));
    std::vector<const void *> vals((size_t)E * 6, nullptr);
    const int64_t I = c.moe_intermediate_size;
    int fmt = -1;
    L->index = li;
    if (m->store) {
        // the store's slots fill the table as experts arrive (all null now)
        fmt = m->store->fmt();
        m->store->set_table(li, (void **)L->experts_dev);
    }
    for (int64_t e = 0; !m->store && e < E; e++) {
        const std::string ep = p + "mlp.experts." + std::to_string(e) + ".";
        const ut_qtensor *g, *u, *d;
        UT_TRY(get_qt(m, ep + "gate_proj.weight", I, H, &g));
        UT_TRY(get_qt(m, ep + "up_proj.weight", I, H, &u));
        UT_TRY(get_qt(m, ep + "down_proj.weight", H, I, &d));
        if (fmt < 0) fmt = g->fmt;
        L->eqt.insert(L->eqt.end(), {g, u, d});
        if (g->fmt != fmt || u->fmt != fmt || d->fmt != fmt) {
            set_error(m->ctx, "layer %lld: experts must share one format", (long long)li);
            return UT_ERR_FORMAT;
        }
        vals[0 * E + e] = g->payload;
        vals[1 * E + e] = u->payload;
        vals[2 * E + e] = d->payload;
        vals[3 * E + e] = g->scales;
        vals[4 * E + e] = u->scales;
        vals[5 * E + e] = d->scales;
    }
    L->expert_fmt = fmt;
    if (!moe_shape_ok(fmt, H, I)) {
        set_error(m->ctx, "experts: hidden %lld / inter %lld unsupported for format %d",
                  (long long)H, (long long)I, fmt);
        return UT_ERR_SHAPE;
    }
    UT_CHECK_HIP(m->ctx, hipMemcpy(L->experts_dev, vals.data(), vals.size() * sizeof(void *),
                                   hipMemcpyHostToDevice));
    void **pp = (void **)L->experts_dev;
    L->experts.gate_w = (const uint8_t *const *)(pp + 0 * E);
    L->experts.up_w = (const uint8_t *const *)(pp + 1 * E);
    L->experts.down_w = (const uint8_t *const *)(pp + 2 * E);
    L->experts.gate_s = (const float *const *)(pp + 3 * E);
    L->experts.up_s = (const float *const *)(pp + 4 * E);
    L->experts.down_s = (const float *const *)(pp + 5 * E);
    return UT_OK;
}

// --------------------------------------------------------- workspace ---
int64_t max_inter(const ut_model *m) {
    int64_t I = m->c.moe_intermediate_size * (m->c.n_shared_experts > 0 ? m->c.n_shared_experts : 1);
    if (m->c.intermediate_size > I) I = m->c.intermediate_size;
    if (m->c.moe_intermediate_size > I) I = m->c.moe_intermediate_size;
    return I;
}

int32_t ws_reserve(ut_session *s, int64_t rows) {
    Workspace &w = s->ws;
    if (rows <= w.rows) return UT_OK;
    ut_model *m = s->m;
    const ut_model_config &c = m->c;
    ut_ctx *ctx = s->ctx;
    const int64_t H = c.hidden_size, heads = c.num_attention_heads;
    const int64_t qh = c.qk_nope_head_dim + c.qk_rope_head_dim, Lr = c.kv_lora_rank;
    const int64_t R = rows < 4 ? 4 : rows;
    const int64_t E = c.n_routed_experts, k = c.num_experts_per_tok;
    int64_t kmax = 2 * H;
    for (int64_t v : {c.q_lora_rank, heads * c.v_head_dim, max_inter(m), Lr})
        if (v > kmax) kmax = v;
    int fmt_hint = UT_FMT_INT4;  // layout sizes are largest for the digit formats
    const int64_t slots_routed = moe_slots(4, k, E, -1);
    size_t moe_bytes = moe_layout(4, k, slots_routed, H, c.moe_intermediate_size, fmt_hint).total;
    for (int f : {UT_FMT_INT8, UT_FMT_F32}) {
        size_t b = moe_layout(4, k, slots_routed, H, c.moe_intermediate_size, f).total;
        if (b > moe_bytes) moe_bytes = b;
    }
    for (int f : {UT_FMT_INT4, UT_FMT_INT8, UT_FMT_F32}) {
        size_t b = moe_layout(4, 1, 1, H, max_inter(m), f).total;
        if (b > moe_bytes) moe_bytes = b;
    }
    // routed experts with the shared expert beside them in the same launches
    for (int fa : {UT_FMT_INT4, UT_FMT_INT8})
        for (int fb : {UT_FMT_INT4, UT_FMT_INT8}) {
            size_t b = moe_layout(4, k, slots_routed, H, c.moe_intermediate_size, fa).total +
                       moe_layout(4, 1, 1, H, max_inter(m), fb).total;
            if (b > moe_bytes) moe_bytes = b;
        }
    ScratchPlan plan;
    auto F = [&](int64_t n) { return plan.add((size_t)n * 4); };
    size_t ix = F(R * H), inorm = F(R * H), iattn = F(R * H), imoe = F(R * H);
    size_t iqa = F(R * (c.q_lora_rank > 0 ? c.q_lora_rank : 1)), iqan = F(R * (c.q_lora_rank > 0 ? c.q_lora_rank : 1));
    size_t iq = F(R * heads * qh), icomp = F(R * (Lr + c.qk_rope_head_dim));
    size_t iqabs = F(R * heads * Lr), iqrope = F(R * heads * c.qk_rope_head_dim + 1);
    size_t iclat = F(R * heads * Lr), ictx = F(R * heads * c.v_head_dim);
    size_t ilog = F(R * c.vocab_size), iemb = F(R * H), icat = F(R * 2 * H);
    size_t irl = F(4 * E), irw = F(4 * k), irid = F(4 * k), iids = F(R), iam = F(2 * R + 1), ierr = F(1);
    size_t ivids = F(8);
    size_t ivmax = F(R * absorb_v_parts(heads, c.v_head_dim)), ivexp = F(R);
    size_t idig = plan.add(matmul_digit_bytes(R, kmax));
    size_t idA = plan.add(matmul_digit_bytes(R, kmax));
    size_t idB = plan.add(matmul_digit_bytes(R, kmax));
    size_t imoes = plan.add(moe_bytes);
    size_t imla = plan.add(mla_scratch_bytes(R < kMlaRowsPerCall ? R : kMlaRowsPerCall, heads, Lr, c.qk_rope_head_dim, s->cap));
    size_t iarg = plan.add(argmax_scratch_bytes(R, c.vocab_size) + 256);
    // the fast-int8 path's MLP and expert rows (four rows at a time): gate,
    // up, h [4][max inter], the choices' outputs [4][k][H] and a shared
    // MLP's [4][H]
    size_t ifast = F(3 * 4 * max_inter(m) + 4 * (k > 0 ? k : 1) * H + 4 * H);
    size_t total = 0;
    for (size_t b : plan.sizes) total += b;
    if (w.base) {
        UT_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
        UT_CHECK_HIP(ctx, hipFree(w.base));
        w.base = nullptr;
    }
    // a captured step names the old workspace
    for (auto &g : s->gd)
        if (g) {
            (void)hipGraphExecDestroy(g);
            g = nullptr;
        }
    if (s->gv) {
        (void)hipGraphExecDestroy(s->gv);
        s->gv = nullptr;
    }
    if (s->g1) {
        (void)hipGraphExecDestroy(s->g1);
        s->g1 = nullptr;
    }
    if (hipMalloc(&w.base, total) != hipSuccess) {
        (void)hipGetLastError();
        set_error(ctx, "workspace allocation of %zu bytes failed", total);
        w.rows = 0;
        return UT_ERR_OOM;
    }
    w.bytes = total;
    std::vector<char *> p;
    char *q = (char *)w.base;
    for (size_t b : plan.sizes) { p.push_back(q); q += b; }
    w.x = (float *)p[ix]; w.normed = (float *)p[inorm]; w.attn = (float *)p[iattn];
    w.moe_out = (float *)p[imoe]; w.qa = (float *)p[iqa]; w.qa_n = (float *)p[iqan];
    w.q = (float *)p[iq]; w.comp = (float *)p[icomp]; w.qabs = (float *)p[iqabs];
    w.qrope = (float *)p[iqrope]; w.clat = (float *)p[iclat]; w.ctxv = (float *)p[ictx];
    w.logits = (float *)p[ilog]; w.emb = (float *)p[iemb]; w.cat = (float *)p[icat];
    w.rlogits = (float *)p[irl]; w.rw = (float *)p[irw]; w.rids = (int32_t *)p[irid];
    w.ids = (int32_t *)p[iids]; w.am = (int32_t *)p[iam]; w.err = (int32_t *)p[ierr];
    w.vids = (int32_t *)p[ivids];
    w.vmax = (uint32_t *)p[ivmax]; w.vexps = (int32_t *)p[ivexp];
    w.digits = p[idig]; w.moe = p[imoes]; w.mla = p[imla]; w.argm = p[iarg];
    w.digA = p[idA]; w.digB = p[idB];
    w.fast = (float *)p[ifast];
    w.rows = R;
    UT_CHECK_HIP(ctx, hipMemsetAsync(w.err, 0, 4, ctx->stream));
    return UT_OK;
}

// ------------------------------------------------------------ forward ---
int32_t mm(ut_session *s, const ut_qtensor *w, const float *x, int64_t M, float *out, int64_t ldo,
           int accumulate = 0) {
    return matmul_dev(s->ctx, w, x, M, out, ldo, accumulate, s->ws.digits);
}

// The opt-in fast-int8 mode (ut_set_fast_int8 on the session's context,
// undertow-quant/src/lib.rs:31-59): every int8 QTensor::matmul of the model
// quantises its activations per row (matmul_dev / matmul_digits take the
// fast kernel), so the fused launches that hand digits between kernels are
// not used, and the MLPs and routed experts run as separate matmuls in the
// reference's order.
bool fast8(const ut_session *s) { return s->ctx->fast_int8; }

// h = silu(g) * u (undertow-quant/src/lib.rs:121, model.rs:241-247)
__global__ void k_silu_mul(const float *__restrict__ g, const float *__restrict__ u,
                           float *__restrict__ h, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float gv = g[i];
    h[i] = __fmul_rn(gv / (1.0f + expf(-gv)), u[i]);
}

// out[s] (+)= (init[s] +) y[s] per element: forward_add of an MLP, or with
// init the shared expert added to the routed sum before the residual add
__global__ void k_add_rows(float *__restrict__ out, int64_t ldo, const float *__restrict__ init,
                           const float *__restrict__ y, int64_t n, int64_t rows) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n * rows) return;
    const int64_t r = i / n, o = i - r * n;
    const float t = init ? __fadd_rn(init[r * n + o], y[i]) : y[i];
    float *po = out + r * ldo + o;
    *po = __fadd_rn(*po, t);
}

// moe_forward's combine (model.rs:268-284) over per-choice outputs
// d [rows][k][H]: sum = 0, sum += w[s,c] * d[s,c] in router order (choices
// with a negative id skipped), then + shared[s] when given, then the
// residual add out[s] += sum.
__global__ void k_combine_rows(const float *__restrict__ d, const float *__restrict__ w,
                               const int32_t *__restrict__ ids, int k, int64_t H,
                               const float *__restrict__ shared, float *__restrict__ out,
                               int64_t ldo) {
    const int s = blockIdx.y;
    const int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (o >= H) return;
    float acc = 0.0f;
    for (int c = 0; c < k; c++) {
        if (ids[s * k + c] < 0) continue;
        acc = __fadd_rn(acc, __fmul_rn(w[s * k + c], d[((int64_t)s * k + c) * H + o]));
    }
    if (shared) acc = __fadd_rn(acc, shared[(int64_t)s * H + o]);
    float *po = out + (int64_t)s * ldo + o;
    *po = __fadd_rn(*po, acc);
}

// An MLP over up to four rows as three matmuls (MlpWeights::forward_add,
// model.rs:43-58): y = down(silu(gate x) * up x), then out += y, or with
// init out += init + y.  y_out: also keep y there (the shared expert).
int32_t mlp_rows_fast(ut_session *s, const MlpW &w, const float *x, int64_t rows, float *out,
                      int64_t ldo, const float *init, float *y_out) {
    ut_ctx *ctx = s->ctx;
    const int64_t H = hd(s->m), I = w.inter, R = max_inter(s->m);
    const int64_t k = s->m->c.num_experts_per_tok > 0 ? s->m->c.num_experts_per_tok : 1;
    // ws.fast: g, u, h [4][R], then the choices' outputs [4][k][H], then y [4][H]
    float *g = s->ws.fast, *u = g + 4 * R, *h = u + 4 * R, *y = h + 4 * R + 4 * k * H;
    UT_TRY(mm(s, w.gate, x, rows, g, I));
    UT_TRY(mm(s, w.up, x, rows, u, I));
    const int64_t n = rows * I;
    hipLaunchKernelGGL(k_silu_mul, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, ctx->stream, g, u,
                       h, n);
    UT_TRY(launch_check(ctx, "k_silu_mul"));
    if (y_out) return mm(s, w.down, h, rows, y_out, H);
    if (!init) return mm(s, w.down, h, rows, out, ldo, 1);
    UT_TRY(mm(s, w.down, h, rows, y, H));
    hipLaunchKernelGGL(k_add_rows, dim3((unsigned)((rows * H + 255) / 256)), dim3(256), 0,
                       ctx->stream, out, ldo, init, y, H, rows);
    return launch_check(ctx, "k_add_rows");
}

// Digit forms the given weights need from one shared activation.
int dig_flags(std::initializer_list<const ut_qtensor *> ws) {
    int f = 0;
    for (const ut_qtensor *w : ws) {
        if (!w || w->fmt == UT_FMT_F32) continue;
        const bool fast = (w->fmt == UT_FMT_INT4 ? w->in_dim % 32 == 0 : w->in_dim % 16 == 0) &&
                          ((uintptr_t)w->payload & 15) == 0;
        f |= fast ? xdigit_flags_for(w->fmt, w->in_dim) : XD_XT;
    }
    return f;
}

// Whether any of the weights reads its activation as f32 (f32 weights:
// the integer formats read digits only).
bool f32_reader(std::initializer_list<const ut_qtensor *> ws) {
    for (const ut_qtensor *w : ws)
        if (w && w->fmt == UT_FMT_F32) return true;
    return false;
}

int dig_flags_fmt(int fmt, int64_t K) {
    if (fmt == UT_FMT_F32) return 0;
    return xdigit_flags_for(fmt, K);
}

// rmsnorm rows of x into out (f32) and into digits in `buf` for consumers
// needing `flags`.
int32_t norm_dig(ut_session *s, const float *x, int64_t ldx, const float *w, int64_t n,
                 int64_t rows, float *out, int64_t ldo, void *buf, int flags, XDigits *xd) {
    const ut_model_config &c = s->m->c;
    *xd = xdigits_view(buf, rows, n, flags);
    return launch_rmsnorm_digitize(s->ctx, x, ldx, rows, n, w, c.rms_norm_eps, out, ldo, *xd,
                                   flags);
}

// An MLP (dense FFN or shared expert) over rows, added into out
// (MlpWeights::forward_add, model.rs:43-58).  xd: digits of x.  With init,
// out = out + (init + mlp(x)) instead (the shared expert added to the routed
// sum, then the residual add, in the reference's order).
int32_t mlp_add(ut_session *s, const MlpW &w, const float *x, const XDigits &xd, int64_t rows,
                float *out, const float *init = nullptr, const NormNext *next = nullptr) {
    ut_model *m = s->m;
    if (next && rows > 4) return UT_ERR_ARG;  // x and xd would be overwritten mid-loop
    if (fast8(s)) {
        if (next) return UT_ERR_ARG;  // the fused next norm is not used in this mode
        const int64_t H = hd(m);
        for (int64_t s0 = 0; s0 < rows; s0 += 4)
            UT_TRY(mlp_rows_fast(s, w, x + s0 * H, rows - s0 < 4 ? rows - s0 : 4, out + s0 * H, H,
                                 init ? init + s0 * H : nullptr, nullptr));
        return UT_OK;
    }
    for (int64_t s0 = 0; s0 < rows; s0 += 4) {
        MoeCall c;
        c.fmt = w.fmt;
        c.tbl = w.ptrs;
        c.E = 1;
        c.H = hd(m);
        c.I = w.inter;
        c.M = (int)(rows - s0 < 4 ? rows - s0 : 4);
        c.k = 1;
        c.ids = m->zeros;
        c.weights = m->ones;
        c.x = x + s0 * c.H;
        XDigits xr = xdigits_rows(xd, s0);
        if (w.fmt != UT_FMT_F32) c.x_digits = &xr;
        c.out = out + s0 * c.H;
        c.ldo = c.H;
        c.accumulate = 1;
        c.err_flag = s->ws.err;
        MoePlan mp = m->mlp_plan;
        mp.sp = (const void **)w.dev;  // the MLP's 6 weight pointers are its slot 0
        c.plan = &mp;
        c.init = init ? init + s0 * c.H : nullptr;
        c.next = next;
        UT_TRY(moe_pass(s->ctx, c, s->ws.moe));
    }
    return UT_OK;
}

// The routed experts of M rows through the HBM tier: the choices (and, at
// one row with pilot hints on, the next MoE layer's predicted choices:
// pilot_prefetch, model.rs:290-318, on the post-attention residual `resid`)
// come back to the host in one round trip; missing experts are loaded into
// slots and the layer's pointer table published, all in stream order.
int32_t tiered_experts(ut_session *s, const LayerW &L, const float *resid, int64_t M) {
    ut_model *m = s->m;
    ut_ctx *ctx = s->ctx;
    const ut_model_config &c = m->c;
    const int64_t E = c.n_routed_experts, k = c.num_experts_per_tok, H = c.hidden_size;
    const int64_t n = M * k;
    const LayerW *nxt = nullptr;
    if (m->store_prefetch && M == 1 && L.index + 1 < c.num_hidden_layers &&
        !m->layers[(size_t)L.index + 1].dense)
        nxt = &m->layers[(size_t)L.index + 1];
    if (nxt) {
        // row 1 of the workspace's router buffers is free at one row
        UT_TRY(launch_rmsnorm(ctx, resid, H, nxt->post_norm, H, c.rms_norm_eps, 1, s->ws.emb, H));
        UT_TRY(mm(s, nxt->gate, s->ws.emb, 1, s->ws.rlogits + E, E));
        UT_TRY(launch_route(ctx, s->ws.rlogits + E, nxt->bias, 1, E, (int)k, (int)c.n_group,
                            (int)c.topk_group, c.norm_topk_prob, c.routed_scaling_factor,
                            s->ws.rids + k, s->ws.rw + k));
    }
    const int64_t nb = nxt ? n + k : n;
    std::vector<int32_t> ids((size_t)nb);
    // through the context's pinned buffer: the session's readback slot may
    // hold a generation loop's token still to be read
    void *pin = nullptr;
    UT_TRY(pinned_acquire(ctx, (size_t)nb * 4, &pin));
    UT_CHECK_HIP(ctx, hipMemcpyAsync(pin, s->ws.rids, (size_t)nb * 4, hipMemcpyDeviceToHost,
                                     ctx->stream));
    UT_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    memcpy(ids.data(), pin, (size_t)nb * 4);
    UT_TRY(m->store->ensure(L.index, ids.data(), n));
    if (nxt) UT_TRY(m->store->prefetch(nxt->index, ids.data() + n, k));
    return UT_OK;
}

// The routed part of moe_forward (model.rs:195-281): router, routed experts
// in choice order, into out (overwritten).  x: normed rows (f32, for the f32
// router gate) with digits xd.
int32_t moe_forward(ut_session *s, const LayerW &L, const float *x, const XDigits &xd,
                    int64_t rows, float *out, int accumulate = 0, const MlpW *shared = nullptr,
                    const NormNext *next = nullptr) {
    ut_model *m = s->m;
    const ut_model_config &c = m->c;
    if (next && rows > 4) return UT_ERR_ARG;  // x and xd would be overwritten mid-loop
    const int64_t H = c.hidden_size, E = c.n_routed_experts;
    const int k = (int)c.num_experts_per_tok;
    for (int64_t s0 = 0; s0 < rows; s0 += 4) {
        const int M = (int)(rows - s0 < 4 ? rows - s0 : 4);
        // f32 gate matmul (lib.rs:128), then route (router.rs:58) + slot plan;
        // a split gate GEMV leaves its partials to the router launch
        SplitKPartials gparts;
        {
            GemvArgs ga;
            ga.w = L.gate;
            ga.xf = x + s0 * H;
            ga.M = M;
            ga.out = s->ws.rlogits;
            ga.ldo = E;
            // the tiered path routes in its own launch: logits finished here
            ga.defer = m->store ? nullptr : &gparts;
            if (L.gate->fmt != UT_FMT_F32) {
                UT_TRY(mm(s, L.gate, x + s0 * H, M, s->ws.rlogits, E));
                gparts = SplitKPartials{};
            } else if (rowdot_f32_ok(L.gate, M) && ((uintptr_t)(x + s0 * H) & 15) == 0) {
                UT_TRY(launch_rowdot_f32(s->ctx, L.gate, x + s0 * H, M, s->ws.rlogits, E));
                gparts = SplitKPartials{};
            } else {
                UT_TRY(gemv(s->ctx, ga));
            }
        }
        const int64_t slots = moe_slots(M, k, E, -1);
        ScratchLayout lay = moe_layout(M, k, slots, H, c.moe_intermediate_size, L.expert_fmt);
        if (m->store) {
            // the HBM tier: route, read the choices back, bring missing
            // experts into their slots (TieredStore::get_expert), then the
            // expert launches plan from the ids like a resident table
            UT_TRY(launch_route(s->ctx, s->ws.rlogits, L.bias, M, E, k, (int)c.n_group,
                                (int)c.topk_group, c.norm_topk_prob, c.routed_scaling_factor,
                                s->ws.rids, s->ws.rw));
            UT_TRY(tiered_experts(s, L, s->ws.x + s0 * H, M));
        }
        // with the logits whole and few choices the expert launch routes and
        // builds the slot plan itself (moe_pass); else route + plan in one
        // launch here
        // (two or more rows go to the matrix-core expert kernels, which take
        // the plan ready-made: route and plan in one launch)
        const bool mfma_rows = M >= 2 && gate_up_mfma_ok(L.expert_fmt, M, H);
        const bool gate_plans = !m->store && gparts.ks <= 1 && (int64_t)M * k <= 64 &&
                                L.expert_fmt != UT_FMT_F32 && !mfma_rows;
        if (!gate_plans && !m->store)
            UT_TRY(launch_route_plan(s->ctx, s->ws.rlogits, &gparts, L.bias, M, E, k,
                                     (int)c.n_group, (int)c.topk_group, c.norm_topk_prob,
                                     c.routed_scaling_factor, s->ws.rids, s->ws.rw,
                                     (const void *const *)L.experts.gate_w,
                                     moe_plan_view(s->ws.moe, lay), s->ws.err));
        MoeCall mc;
        mc.fmt = L.expert_fmt;
        mc.tbl = L.experts;
        mc.E = E;
        mc.H = H;
        mc.I = c.moe_intermediate_size;
        mc.M = M;
        mc.k = k;
        mc.ids = s->ws.rids;
        mc.weights = s->ws.rw;
        mc.x = x + s0 * H;
        XDigits xr = xdigits_rows(xd, s0);
        if (L.expert_fmt != UT_FMT_F32) mc.x_digits = &xr;
        mc.x_matches_digits = true;  // xd digitised exactly these rows of x
        mc.out = out + s0 * H;
        mc.ldo = H;
        mc.accumulate = accumulate;
        mc.err_flag = s->ws.err;
        mc.plan_ready = !gate_plans && !m->store;
        if (gate_plans) {
            mc.route_logits = s->ws.rlogits;
            mc.route_bias = L.bias;
            mc.route_ng = (int)c.n_group;
            mc.route_tg = (int)c.topk_group;
            mc.route_norm = c.norm_topk_prob;
            mc.route_scale = c.routed_scaling_factor;
            mc.route_ids = s->ws.rids;
            mc.route_w = s->ws.rw;
        }
        MoeCall sc;
        MoePlan sp_plan = m->mlp_plan;
        if (shared) {
            sc.fmt = shared->fmt;
            sc.tbl = shared->ptrs;
            sc.I = shared->inter;
            sp_plan.sp = (const void **)shared->dev;  // slot 0 = the shared expert
            sc.plan = &sp_plan;
            mc.shared = &sc;
            mc.shared_scratch = (char *)s->ws.moe + lay.total;
        }
        mc.next = next;
        UT_TRY(moe_pass(s->ctx, mc, s->ws.moe));
    }
    return UT_OK;
}

// moe_forward in the fast-int8 mode (model.rs:195-286) over normed rows x,
// added with the shared expert into out (the residual): the f32 router
// gate and the router on the device, the choices read back, each choice's
// expert MLP as three matmuls of its row (activations are quantised per
// row, so a row's result does not depend on which rows share an expert),
// then the combine in router order.
int32_t moe_forward_fast(ut_session *s, const LayerW &L, const float *x, int64_t rows, float *out) {
    ut_model *m = s->m;
    ut_ctx *ctx = s->ctx;
    const ut_model_config &c = m->c;
    if (m->store || L.eqt.empty()) {
        set_error(ctx, "the fast-int8 mode needs every routed expert resident");
        return UT_ERR_STATE;
    }
    const int64_t H = c.hidden_size, E = c.n_routed_experts, I = c.moe_intermediate_size;
    const int k = (int)c.num_experts_per_tok;
    const int64_t R = max_inter(m);
    float *d = s->ws.fast + 3 * 4 * R, *ysh = d + 4 * k * H;
    for (int64_t s0 = 0; s0 < rows; s0 += 4) {
        const int M = (int)(rows - s0 < 4 ? rows - s0 : 4);
        UT_TRY(mm(s, L.gate, x + s0 * H, M, s->ws.rlogits, E));
        UT_TRY(launch_route(ctx, s->ws.rlogits, L.bias, M, E, k, (int)c.n_group, (int)c.topk_group,
                            c.norm_topk_prob, c.routed_scaling_factor, s->ws.rids, s->ws.rw));
        std::vector<int32_t> ids((size_t)M * k);
        void *pin = nullptr;
        UT_TRY(pinned_acquire(ctx, ids.size() * 4, &pin));
        UT_CHECK_HIP(ctx, hipMemcpyAsync(pin, s->ws.rids, ids.size() * 4, hipMemcpyDeviceToHost,
                                         ctx->stream));
        UT_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
        memcpy(ids.data(), pin, ids.size() * 4);
        for (int r = 0; r < M; r++)
            for (int j = 0; j < k; j++) {
                const int32_t e = ids[(size_t)r * k + j];
                if (e < 0) continue;
                if (e >= E) {
                    set_error(ctx, "a routed expert id was out of range or not loaded");
                    return UT_ERR_BAD_EXPERT;
                }
                MlpW ew;
                ew.gate = L.eqt[(size_t)3 * e];
                ew.up = L.eqt[(size_t)3 * e + 1];
                ew.down = L.eqt[(size_t)3 * e + 2];
                ew.fmt = ew.gate->fmt;
                ew.inter = I;
                UT_TRY(mlp_rows_fast(s, ew, x + (s0 + r) * H, 1, nullptr, 0, nullptr,
                                     d + ((int64_t)r * k + j) * H));
            }
        if (L.has_shared)
            UT_TRY(mlp_rows_fast(s, L.shared, x + s0 * H, M, nullptr, 0, nullptr, ysh));
        hipLaunchKernelGGL(k_combine_rows, dim3((unsigned)((H + 255) / 256), (unsigned)M), dim3(256),
                           0, ctx->stream, d, s->ws.rw, s->ws.rids, k, H,
                           L.has_shared ? ysh : nullptr, out + s0 * H, H);
        UT_TRY(launch_check(ctx, "k_combine_rows"));
    }
    return UT_OK;
}

// mla_forward_cached, absorbed form (attention.rs:123-279), added into out
// (the residual).  x: normed rows with digits xd.
int32_t mla_forward(ut_session *s, const LayerW &L, const float *x, const XDigits &xd,
                    int64_t rows, KvCache &kv, float *out, const NormNext *post = nullptr,
                    bool *post_done = nullptr) {
    if (post_done) *post_done = false;
    ut_model *m = s->m;
    ut_ctx *ctx = s->ctx;
    const ut_model_config &c = m->c;
    Workspace &w = s->ws;
    const int64_t heads = c.num_attention_heads, nope = c.qk_nope_head_dim,
                  rope = c.qk_rope_head_dim, vh = c.v_head_dim, Lr = c.kv_lora_rank;
    const int64_t qh = nope + rope;
    const float scale = 1.0f / sqrtf((float)qh);  // config.rs:142-144
    const int64_t pos_base = kv.len;
    const bool pair = !fast8(s) && L.lora && L.kv_a->fmt == L.q_a->fmt && L.kv_a->fmt != UT_FMT_F32 &&
                      L.kv_a->in_dim == L.q_a->in_dim && L.kv_a->row_bytes == L.q_a->row_bytes &&
                      gemv_fast_ok(L.kv_a) && gemv_fast_ok(L.q_a);
    // with the pair's split-K partials deferred, one launch finishes both
    // outputs: q_a's norm + digits and kv_a's cache append
    const bool fused = pair && mla_pre_ok(rows, c.q_lora_rank, Lr, rope);
    SplitKPartials pp;
    // one or two rows: the pair's rows finished in their workgroups (K split
    // inside them), q_b normalising q_a while staging it and, in one more
    // workgroup per row of its launch, the kv appends -- no mla_pre launch
    GemvArgs pa;
    pa.w = L.kv_a;
    pa.xf = x;
    pa.xd = xd;
    pa.M = rows;
    pa.out = w.comp;
    pa.ldo = Lr + rope;
    pa.w2 = L.q_a;
    pa.out2 = w.qa;
    pa.ldo2 = c.q_lora_rank;
    const bool rowsplit = fused && rows <= 2 && gemv_rowsplit_ok(pa) &&
                          gemv_norm_ok(L.q_b, rows, w.qa, L.q_a_norm);
    if (rowsplit) {
        UT_TRY(launch_gemv_rowsplit(ctx, pa));
        KvAppendArgs kva;
        kva.comp = w.comp;
        kva.L = Lr;
        kva.P = rope;
        kva.w = L.kv_a_norm;
        kva.eps = c.rms_norm_eps;
        kva.latent = kv.latent;
        kva.krot = kv.krot;
        kva.kc = kv.kc;
        kva.pos = pos_ref(ctx, pos_base);
        kva.table = m->rope_table;
        GemvArgs gq;
        gq.w = L.q_b;
        gq.M = rows;
        gq.xf = w.qa;
        gq.out = w.q;
        gq.ldo = heads * qh;
        gq.norm_w = L.q_a_norm;
        gq.norm_eps = c.rms_norm_eps;
        gq.kv = &kva;
        UT_TRY(gemv(ctx, gq));
    } else if (pair) {
        // kv_a and q_a read the same normed row: one launch for both
        GemvArgs ga;
        ga.w = L.kv_a;
        ga.xf = x;
        ga.xd = xd;
        ga.M = rows;
        ga.out = w.comp;
        ga.ldo = Lr + rope;
        ga.w2 = L.q_a;
        ga.out2 = w.qa;
        ga.ldo2 = c.q_lora_rank;
        if (fused) ga.defer = &pp;
        UT_TRY(gemv(ctx, ga));
    } else {
        UT_TRY(matmul_digits(ctx, L.kv_a, x, xd, rows, w.comp, Lr + rope, 0));
    }
    // one row: q_b normalises q_a itself while staging it (the same digits
    // as the row digitiser's), so mla_pre only sums q_a's partials
    const bool qb_norm = !rowsplit && fused && pp.ks > 1 && rows == 1 &&
                         gemv_norm_ok(L.q_b, 1, w.qa, L.q_a_norm);
    if (rowsplit) {
        // done above
    } else if (qb_norm) {
        UT_TRY(launch_mla_pre(ctx, pp, Lr + rope, xd.exps, L.kv_a->scales, L.q_a->scales, rows,
                              c.q_lora_rank, L.q_a_norm, c.rms_norm_eps, nullptr, XDigits{}, 0, Lr,
                              rope, L.kv_a_norm, kv.latent, kv.krot, kv.kc, pos_base,
                              m->rope_table, w.qa));
        GemvArgs gq;
        gq.w = L.q_b;
        gq.M = 1;
        gq.xf = w.qa;
        gq.out = w.q;
        gq.ldo = heads * qh;
        gq.norm_w = L.q_a_norm;
        gq.norm_eps = c.rms_norm_eps;
        UT_TRY(gemv(ctx, gq));
    } else if (fused && pp.ks > 1) {
        const int qf = dig_flags({L.q_b});
        const XDigits qd = xdigits_view(w.digB, rows, c.q_lora_rank, qf);
        UT_TRY(launch_mla_pre(ctx, pp, Lr + rope, xd.exps, L.kv_a->scales, L.q_a->scales, rows,
                              c.q_lora_rank, L.q_a_norm, c.rms_norm_eps,
                              f32_reader({L.q_b}) ? w.qa_n : nullptr, qd, qf, Lr, rope,
                              L.kv_a_norm, kv.latent, kv.krot, kv.kc, pos_base, m->rope_table));
        UT_TRY(matmul_digits(ctx, L.q_b, w.qa_n, qd, rows, w.q, heads * qh, 0));
    } else {
        if (L.lora) {
            if (!pair) UT_TRY(matmul_digits(ctx, L.q_a, x, xd, rows, w.qa, c.q_lora_rank, 0));
            XDigits qd;
            UT_TRY(norm_dig(s, w.qa, c.q_lora_rank, L.q_a_norm, c.q_lora_rank, rows, w.qa_n,
                            c.q_lora_rank, w.digB, dig_flags({L.q_b}), &qd));
            UT_TRY(matmul_digits(ctx, L.q_b, w.qa_n, qd, rows, w.q, heads * qh, 0));
        } else {
            UT_TRY(matmul_digits(ctx, L.q_proj, x, xd, rows, w.q, heads * qh, 0));
        }
        UT_TRY(launch_kv_append(ctx, w.comp, rows, Lr, rope, L.kv_a_norm, c.rms_norm_eps,
                                kv.latent, kv.krot, kv.kc, pos_base, m->rope_table));
    }
    kv.len = pos_base + rows;
    UT_TRY(launch_absorb_q(ctx, L.kv_b, w.q, rows, heads, nope, rope, vh, w.qabs, w.qrope,
                           pos_base, m->rope_table));
    // query rows in groups of kMlaRowsPerCall (bounded scratch; a row's
    // result does not depend on its group)
    for (int64_t r0 = 0; r0 < rows; r0 += kMlaRowsPerCall) {
        const int64_t rn = rows - r0 < kMlaRowsPerCall ? rows - r0 : kMlaRowsPerCall;
        if (kv.kc)
            UT_TRY(launch_mla_attend_kc(ctx, w.qabs + r0 * heads * Lr, w.qrope + r0 * heads * rope,
                                        kv.kc, rn, heads, Lr, rope, pos_base + r0, scale,
                                        w.clat + r0 * heads * Lr, w.mla));
        else
            UT_TRY(launch_mla_attend(ctx, w.qabs + r0 * heads * Lr, w.qrope + r0 * heads * rope,
                                     kv.latent, kv.krot, rn, heads, Lr, rope, pos_base + r0, scale,
                                     w.clat + r0 * heads * Lr, w.mla));
    }
    // x += o_proj(ctx) (the residual add of model.rs:478-480 in the epilogue);
    // with absorb_v's row maxima the o_proj GEMV digitises ctx itself while
    // staging (no separate digitising launch; the same digits)
    const bool vm = !fast8(s) && absorb_v_max_ok(L.kv_b) && L.o_proj->fmt != UT_FMT_F32 &&
                    gemv_fast_ok(L.o_proj) && rows <= 4;
    UT_TRY(launch_absorb_v(ctx, L.kv_b, w.clat, rows, heads, nope, vh, w.ctxv,
                           vm ? w.vmax : nullptr));
    if (!vm) return mm(s, L.o_proj, w.ctxv, rows, out, c.hidden_size, 1);
    GemvArgs ga;
    ga.w = L.o_proj;
    ga.M = rows;
    ga.xf = w.ctxv;
    ga.out = out;
    ga.ldo = c.hidden_size;
    ga.accumulate = 1;
    ga.xmax = w.vmax;
    ga.nxmax = (int)absorb_v_parts(heads, vh);
    ga.exps_out = w.vexps;
    // the post-attention norm runs in o_proj's partial sum when K is split
    ga.next = post;
    ga.next_done = post_done;
    return gemv(ctx, ga);
}

// Whether the norm that follows a layer (the next layer's input norm, the
// final norm) can run inside the layer's last combine: every consumer of the
// layer's own normed rows has run by then, and rows fit one combine.
bool fuse_next_ok(const ut_session *s, int64_t rows) {
    return rows <= 4 && moe_combine_norm_ok(s->m->c.hidden_size) && !fast8(s);
}

// The fused norm's arguments: rmsnorm with norm_w into ws.normed (only when
// a consumer reads the normed rows as f32: f32) and the digit forms `flags`
// into ws.digA; *xd gets the view the consumers read.
NormNext next_norm(ut_session *s, const float *norm_w, int flags, int64_t rows, XDigits *xd,
                   bool f32 = true) {
    const int64_t H = s->m->c.hidden_size;
    NormNext nx;
    nx.norm_w = norm_w;
    nx.eps = s->m->c.rms_norm_eps;
    nx.normed = f32 ? s->ws.normed : nullptr;
    nx.ldn = H;
    nx.flags = flags;
    nx.nd = *xd = xdigits_view(s->ws.digA, rows, H, flags);
    return nx;
}

int input_flags(const LayerW &L) { return dig_flags({L.q_a, L.q_proj, L.kv_a}); }
bool input_f32(const LayerW &L) { return f32_reader({L.q_a, L.q_proj, L.kv_a}); }

// run_layer (model.rs:127-183) / the per-layer body of prefill (:470-526).
// pre: the input norm already ran (its rows in ws.normed, digits *pre).
// next: the following norm, run by the layer's last combine.
int32_t run_layer(ut_session *s, const LayerW &L, float *x, int64_t rows, KvCache &kv,
                  const XDigits *pre = nullptr, const NormNext *next = nullptr) {
    ut_model *m = s->m;
    ut_ctx *ctx = s->ctx;
    const ut_model_config &c = m->c;
    const int64_t H = c.hidden_size;
    Workspace &w = s->ws;
    XDigits xd;
    if (pre) xd = *pre;
    else UT_TRY(norm_dig(s, x, H, L.input_norm, H, rows, w.normed, H, w.digA, input_flags(L), &xd));
    int f = 0;
    if (L.dense) f = dig_flags_fmt(L.mlp.fmt, H);
    else {
        f = dig_flags_fmt(L.expert_fmt, H);
        if (L.has_shared) f |= dig_flags_fmt(L.shared.fmt, H);
    }
    // the post-attention norm, run inside o_proj's split-K sum where it can
    // be (every reader of the layer's normed input has run by then)
    XDigits pd;
    const NormNext post = next_norm(s, L.post_norm, f, rows, &pd);
    bool post_done = false;
    UT_TRY(mla_forward(s, L, w.normed, xd, rows, kv, x, fuse_next_ok(s, rows) ? &post : nullptr,
                       &post_done));
    if (post_done) xd = pd;
    else UT_TRY(norm_dig(s, x, H, L.post_norm, H, rows, w.normed, H, w.digA, f, &xd));
    if (L.dense) return mlp_add(s, L.mlp, w.normed, xd, rows, x, nullptr, next);
    if (fast8(s)) return moe_forward_fast(s, L, w.normed, rows, x);
    // x += (routed + shared) (model.rs:282-284 then the residual add)
    if (L.has_shared && moe_dual_ok(L.expert_fmt, L.shared.fmt))
        return moe_forward(s, L, w.normed, xd, rows, x, 1, &L.shared, next);
    if (!L.has_shared) return moe_forward(s, L, w.normed, xd, rows, x, 1, nullptr, next);
    UT_TRY(moe_forward(s, L, w.normed, xd, rows, w.moe_out));
    return mlp_add(s, L.shared, w.normed, xd, rows, x, w.moe_out, next);
}

int32_t check_flags(ut_session *s) {
    // called after a stream sync: the sticky expert-id error flag
    ut_ctx *ctx = s->ctx;
    int32_t f = 0;
    UT_CHECK_HIP(ctx, hipMemcpy(&f, s->ws.err, 4, hipMemcpyDeviceToHost));
    if (f) {
        set_error(ctx, "a routed expert id was out of range or not loaded");
        return UT_ERR_BAD_EXPERT;
    }
    return UT_OK;
}

int32_t upload_ids(ut_session *s, const int32_t *ids, int64_t n) {
    ut_ctx *ctx = s->ctx;
    void *pin = nullptr;
    UT_TRY(pinned_acquire(ctx, (size_t)n * 4, &pin));
    // the pinned buffer may still feed an earlier copy: order behind the stream
    UT_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    memcpy(pin, ids, (size_t)n * 4);
    UT_CHECK_HIP(ctx, hipMemcpyAsync(s->ws.ids, pin, (size_t)n * 4, hipMemcpyHostToDevice, ctx->stream));
    return UT_OK;
}

// InferenceSession::prefill (model.rs:447-547) into ws.logits / ws.am.
// ids_dev: the token ids are already on the device (an earlier argmax:
// always in the vocabulary); they are not checked, uploaded or recorded in
// s->tokens (the caller records them once it has read them back).
int32_t prefill_dev(ut_session *s, const int32_t *ids, int64_t n, const int32_t *ids_dev = nullptr) {
    ut_model *m = s->m;
    ut_ctx *ctx = s->ctx;
    const ut_model_config &c = m->c;
    if (n <= 0) {
        set_error(ctx, "empty prompt");
        return UT_ERR_ARG;
    }
    if (s->pos + n > s->cap) {
        set_error(ctx, "context overflow: %lld + %lld > %lld", (long long)s->pos, (long long)n,
                  (long long)s->cap);
        return UT_ERR_CONTEXT_OVERFLOW;
    }
    if (ids_dev) {
        // device ids point into the workspace: it must not move
        if (n > s->ws.rows) {
            set_error(ctx, "device-fed prefill of %lld rows exceeds the workspace", (long long)n);
            return UT_ERR_STATE;
        }
    } else {
        for (int64_t i = 0; i < n; i++)
            if (ids[i] < 0 || ids[i] >= c.vocab_size) {
                set_error(ctx, "token id %d out of vocab (%lld)", ids[i], (long long)c.vocab_size);
                return UT_ERR_BAD_TOKEN;
            }
        UT_TRY(ws_reserve(s, n));
    }
    Workspace &w = s->ws;
    const int64_t H = c.hidden_size, V = c.vocab_size;
    if (!ids_dev) UT_TRY(upload_ids(s, ids, n));
    // each layer's last combine runs the norm that follows it when the rows
    // fit one combine (decode and verify steps); the first layer's input
    // norm then runs in the embedding lookup's launch
    const bool fuse = fuse_next_ok(s, n);
    XDigits cur, nxt;
    const size_t nl = m->layers.size();
    const bool emb_norm = fuse && nl > 0 && embed_norm_ok(m->embed, H, w.x, m->layers[0].input_norm);
    if (emb_norm) {
        const NormNext n0 = next_norm(s, m->layers[0].input_norm, input_flags(m->layers[0]), n,
                                      &cur, input_f32(m->layers[0]));
        UT_TRY(launch_embed_norm(ctx, m->embed, ids_dev ? ids_dev : w.ids, n, w.x, H, n0));
    } else {
        UT_TRY(launch_embed(ctx, m->embed, ids_dev ? ids_dev : w.ids, n, w.x, H));
    }
    for (size_t li = 0; li < nl; li++) {
        NormNext nx;
        if (fuse)
            nx = li + 1 < nl ? next_norm(s, m->layers[li + 1].input_norm,
                                         input_flags(m->layers[li + 1]), n, &nxt,
                                         input_f32(m->layers[li + 1]))
                             : next_norm(s, m->final_norm, dig_flags({m->lm_head}), n, &nxt,
                                         f32_reader({m->lm_head}));
        if (fuse && li + 1 == nl && m->has_mtp) {
            // the last combine also keeps the finished rows for the MTP head
            nx.raw2 = s->hidden;
            nx.ld2 = H;
            nx.pos2 = pos_ref(ctx, s->pos);
        }
        UT_TRY(run_layer(s, m->layers[li], w.x, n, s->kv[li],
                         fuse && (li > 0 || emb_norm) ? &cur : nullptr, fuse ? &nx : nullptr));
        cur = nxt;
    }
    if (m->has_mtp && !(fuse && nl > 0)) UT_TRY(launch_copy_rows_at(ctx, s->hidden, H, s->pos, w.x, n, H));
    s->pos += n;
    if (!ids_dev) s->tokens.insert(s->tokens.end(), ids, ids + n);
    XDigits fd = cur;
    if (!fuse || nl == 0)
        UT_TRY(norm_dig(s, w.x, H, m->final_norm, H, n, w.normed, H, w.digA,
                        dig_flags({m->lm_head}), &fd));
    // the argmax rows, then the sticky error word at am[n] and, with device
    // ids (a verify step), the rows' ids past the first (its drafts) at
    // am[n + 1 ...]: one readback carries them all
    const int32_t *tail = ids_dev ? ids_dev + 1 : nullptr;
    const int ntail = ids_dev ? (int)(n - 1) : 0;
    if (n <= 4)
        return matmul_digits_argmax(ctx, m->lm_head, w.normed, fd, n, w.logits, w.am, w.argm,
                                    w.err, tail, ntail);
    UT_TRY(matmul_digits(ctx, m->lm_head, w.normed, fd, n, w.logits, V, 0));
    return launch_argmax(ctx, w.logits, n, V, V, w.am, w.argm, w.err, tail, ntail);
}

int32_t read_argmax(ut_session *s, int64_t n, int32_t *out) {
    ut_ctx *ctx = s->ctx;
    void *pin = nullptr;
    UT_TRY(pinned_acquire(ctx, (size_t)n * 4, &pin));
    UT_CHECK_HIP(ctx, hipMemcpyAsync(pin, s->ws.am, (size_t)n * 4, hipMemcpyDeviceToHost, ctx->stream));
    UT_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    UT_TRY(check_flags(s));
    memcpy(out, pin, (size_t)n * 4);
    return UT_OK;
}

// Asynchronous readback for the generation loops: n ints from dev and the
// sticky error flag into the session's pinned readback slot; `ready` is
// recorded behind them, so later launches need not wait for the host.
// How the flag comes back (err): RB_ERR_COPY in a copy of its own,
// RB_ERR_INLINE as dev[n] (the argmax rows of prefill_dev carry it, and
// after it a verify step's drafts: extra).
enum { RB_ERR_COPY, RB_ERR_INLINE };
int32_t readback_enqueue(ut_session *s, const int32_t *dev, int64_t n, int64_t slot_off = 0,
                         int err = RB_ERR_COPY, int64_t extra = 0) {
    ut_ctx *ctx = s->ctx;
    int32_t *back = s->pin + kPinIds;
    if (slot_off + n + 1 + extra > kPinBack - 1) {
        set_error(ctx, "readback of %lld ints exceeds the staging slot", (long long)(n + extra));
        return UT_ERR_ARG;
    }
    const int64_t cnt = (err == RB_ERR_INLINE ? n + 1 : n) + extra;
    UT_CHECK_HIP(ctx, hipMemcpyAsync(back + slot_off, dev, (size_t)cnt * 4, hipMemcpyDeviceToHost, ctx->stream));
    if (err == RB_ERR_COPY) {
        UT_CHECK_HIP(ctx, hipMemcpyAsync(back + kPinBack - 1, s->ws.err, 4, hipMemcpyDeviceToHost, ctx->stream));
        s->err_slot = kPinBack - 1;
    } else if (err == RB_ERR_INLINE) {
        s->err_slot = slot_off + n;
    }
    UT_CHECK_HIP(ctx, hipEventRecord(s->ready, ctx->stream));
    return UT_OK;
}

// Waits for the last readback; out <- the ints at slot_off.
int32_t readback_wait(ut_session *s, int64_t n, int32_t *out, int64_t slot_off = 0) {
    ut_ctx *ctx = s->ctx;
    UT_CHECK_HIP(ctx, hipEventSynchronize(s->ready));
    const int32_t *back = s->pin + kPinIds;
    if (back[s->err_slot]) {
        set_error(ctx, "a routed expert id was out of range or not loaded");
        return UT_ERR_BAD_EXPERT;
    }
    memcpy(out, back + slot_off, (size_t)n * 4);
    return UT_OK;
}

// Host ids to a device buffer through the pinned upload slot.  The caller
// guarantees that the slot's previous upload has completed (the generation
// loops read back, and so wait, after every step).
// Uploads queued in one step use disjoint offsets of the slot.
int32_t upload_slot(ut_session *s, int32_t *dev, const int32_t *ids, int64_t n, int64_t off = 0) {
    ut_ctx *ctx = s->ctx;
    if (off + n > kPinIds) {
        set_error(ctx, "upload of %lld ids exceeds the staging slot", (long long)n);
        return UT_ERR_ARG;
    }
    memcpy(s->pin + off, ids, (size_t)n * 4);
    UT_CHECK_HIP(ctx, hipMemcpyAsync(dev, s->pin + off, (size_t)n * 4, hipMemcpyHostToDevice,
                                     ctx->stream));
    return UT_OK;
}

void truncate_session(ut_session *s, int64_t len) {
    // model.rs:556-564, LayerKvCache::truncate (attention.rs:89-93)
    for (auto &kv : s->kv)
        if (len < kv.len) kv.len = len;
    if (len < s->pos) s->pos = len;
    if ((int64_t)s->tokens.size() > s->pos) s->tokens.resize((size_t)s->pos);
}

// draft_logits (mtp.rs:74-133): feed positions fed..pos-1 to the MTP layer
// and take the argmax of the head's logits for the last one.
// draft_logits on device ids: row ids come from the host (host_ids, rows of
// them), from dev_ids (rows of them, on the device), or, for a chained
// draft, from ws.vids[in_slot] (one row); the draft id goes to
// ws.vids[out_slot] without a host round trip.
int32_t draft_rows_dev(ut_session *s, const int32_t *host_ids, int in_slot,
                       const float *hidden_rows, int64_t rows, int out_slot,
                       const int32_t *dev_ids = nullptr) {
    ut_model *m = s->m;
    ut_ctx *ctx = s->ctx;
    const ut_model_config &c = m->c;
    Workspace &w = s->ws;
    const int64_t H = c.hidden_size, V = c.vocab_size;
    if (rows > w.rows) UT_TRY(ws_reserve(s, rows));
    const int32_t *ids = dev_ids ? dev_ids : in_slot >= 0 ? w.vids + in_slot : nullptr;
    int32_t *draft_dev = w.vids + out_slot;
    if (!dev_ids && in_slot < 0) {
        for (int64_t i = 0; i < rows; i++)
            if (host_ids[i] < 0 || host_ids[i] >= V) {
                set_error(ctx, "token id %d out of vocab (%lld)", host_ids[i], (long long)V);
                return UT_ERR_BAD_TOKEN;
            }
        // a short feed goes through the session's pinned slot (no wait); a
        // long one (the first draft after a long prompt) through a pinned
        // buffer of its size, ordered behind the stream
        if (rows <= kPinIds - 8) UT_TRY(upload_slot(s, w.ids, host_ids, rows));
        else UT_TRY(upload_ids(s, host_ids, rows));
        ids = w.ids;
    }
    NormNext pre_nx;
    XDigits pre_xd;
    bool pre_done = false;
    if (!fast8(s) && m->eh_proj->fmt != UT_FMT_F32 && gemv_fast_ok(m->eh_proj) &&
        mtp_input_ok(H) && rows <= 4) {
        // the embedding and both norms in one launch, which leaves each
        // half's max|v|; eh_proj digitises cat from them while staging it
        UT_TRY(launch_mtp_input(ctx, m->embed, ids, hidden_rows, rows, H, m->enorm, m->hnorm,
                                c.rms_norm_eps, w.cat, w.vmax));
        GemvArgs ga;
        ga.w = m->eh_proj;
        ga.M = rows;
        ga.xf = w.cat;
        ga.out = w.x;
        ga.ldo = H;
        ga.xmax = w.vmax;
        ga.nxmax = 2;
        ga.exps_out = w.vexps;
        // the MTP layer's input norm in eh_proj's split sum where it can run
        if (fuse_next_ok(s, rows)) {
            pre_nx = next_norm(s, m->mtp_layer.input_norm, input_flags(m->mtp_layer), rows, &pre_xd,
                               input_f32(m->mtp_layer));
            ga.next = &pre_nx;
            ga.next_done = &pre_done;
        }
        UT_TRY(gemv(ctx, ga));
    } else {
        UT_TRY(launch_embed(ctx, m->embed, ids, rows, w.emb, H));
        UT_TRY(launch_rmsnorm(ctx, w.emb, H, m->enorm, H, c.rms_norm_eps, rows, w.cat, 2 * H));
        UT_TRY(launch_rmsnorm(ctx, hidden_rows, H, m->hnorm, H, c.rms_norm_eps, rows, w.cat + H, 2 * H));
        UT_TRY(mm(s, m->eh_proj, w.cat, rows, w.x, H));
    }
    XDigits hd_;
    const float *hn = w.normed;
    if (fuse_next_ok(s, rows)) {
        // the layer's last combine normalises every row; the head reads the last
        XDigits all;
        const NormNext nx = next_norm(s, m->mtp_norm, dig_flags({m->mtp_head}), rows, &all,
                                      f32_reader({m->mtp_head}));
        UT_TRY(run_layer(s, m->mtp_layer, w.x, rows, s->mtp_kv, pre_done ? &pre_xd : nullptr, &nx));
        hd_ = xdigits_rows(all, rows - 1);
        hn = w.normed + (rows - 1) * H;
    } else {
        UT_TRY(run_layer(s, m->mtp_layer, w.x, rows, s->mtp_kv));
        UT_TRY(norm_dig(s, w.x + (rows - 1) * H, H, m->mtp_norm, H, 1, w.normed, H, w.digA,
                        dig_flags({m->mtp_head}), &hd_));
    }
    return matmul_digits_argmax(ctx, m->mtp_head, hn, hd_, 1, w.logits, draft_dev, w.argm, nullptr);
}

// ---------------------------------------------------------- synthesis ---
// Counter-based generator (splitmix64 of seed, tensor index, element index):
// every element is a pure function of its coordinates, so any launch shape
// produces the same model.
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ float u01(uint64_t h) {  // (0, 1)
    return ((float)(h >> 40) + 0.5f) * (1.0f / 16777216.0f);
}

__device__ __forceinline__ float normal01(uint64_t key, uint64_t i) {
    const uint64_t h = mix64(key ^ mix64(i));
    const float u1 = u01(h), u2 = u01(mix64(h));
    return sqrtf(-2.0f * logf(u1)) * cosf(6.283185307f * u2);
}

// kind 0: int4 payload bytes (all 16 codes uniform); 1: int8 codes uniform in
// [-127, 127]; 2: per-row scales |N(0,std)|/qmax; 3: f32 N(0, std);
// 4: norm weights 1 + (u - 0.5) * 0.2; 5: bias ramp -0.1 + 0.2 i/(n-1).
__global__ void k_synth(void *dst, int64_t n, int kind, uint64_t key, float a, float b) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        switch (kind) {
        case 0: ((uint8_t *)dst)[i] = (uint8_t)(mix64(key ^ mix64(i)) >> 56); break;
        case 1: ((int8_t *)dst)[i] = (int8_t)((int)((mix64(key ^ mix64(i)) >> 32) % 255u) - 127); break;
        case 2: ((float *)dst)[i] = fabsf(normal01(key, i)) * a / b; break;
        case 3: ((float *)dst)[i] = normal01(key, i) * a; break;
        case 4: ((float *)dst)[i] = 1.0f + (u01(mix64(key ^ mix64(i))) - 0.5f) * 0.2f; break;
        default: ((float *)dst)[i] = -0.1f + 0.2f * (float)i / (n > 1 ? (float)(n - 1) : 1.0f); break;
        }
    }
}

struct SynthItem {
    std::string name;
    int kind;  // 0 matrix, 1 norm vector, 2 bias vector
    int cls;   // matrices: 0 f32 (router gate), 1 dense, 2 expert
    int64_t d0, d1;
};

void synth_layer_list(const ut_model_config &c, int64_t li, bool dense, std::vector<SynthItem> &v) {
    const int64_t H = c.hidden_size, heads = c.num_attention_heads;
    const int64_t qh = c.qk_nope_head_dim + c.qk_rope_head_dim;
    const std::string p = "model.layers." + std::to_string(li) + ".";
    v.push_back({p + "input_layernorm.weight", 1, 0, H, 1});
    v.push_back({p + "post_attention_layernorm.weight", 1, 0, H, 1});
    if (c.q_lora_rank > 0) {
        v.push_back({p + "self_attn.q_a_proj.weight", 0, 1, c.q_lora_rank, H});
        v.push_back({p + "self_attn.q_a_layernorm.weight", 1, 0, c.q_lora_rank, 1});
        v.push_back({p + "self_attn.q_b_proj.weight", 0, 1, heads * qh, c.q_lora_rank});
    } else {
        v.push_back({p + "self_attn.q_proj.weight", 0, 1, heads * qh, H});
    }
    v.push_back({p + "self_attn.kv_a_proj_with_mqa.weight", 0, 1, c.kv_lora_rank + c.qk_rope_head_dim, H});
    v.push_back({p + "self_attn.kv_a_layernorm.weight", 1, 0, c.kv_lora_rank, 1});
    v.push_back({p + "self_attn.kv_b_proj.weight", 0, 1, heads * (c.qk_nope_head_dim + c.v_head_dim), c.kv_lora_rank});
    v.push_back({p + "self_attn.o_proj.weight", 0, 1, H, heads * c.v_head_dim});
    if (dense) {
        v.push_back({p + "mlp.gate_proj.weight", 0, 1, c.intermediate_size, H});
        v.push_back({p + "mlp.up_proj.weight", 0, 1, c.intermediate_size, H});
        v.push_back({p + "mlp.down_proj.weight", 0, 1, H, c.intermediate_size});
        return;
    }
    const int64_t E = c.n_routed_experts, I = c.moe_intermediate_size;
    v.push_back({p + "mlp.gate.weight", 0, 0, E, H});
    v.push_back({p + "mlp.gate.e_score_correction_bias", 2, 0, E, 1});
    for (int64_t e = 0; e < E; e++) {
        const std::string ep = p + "mlp.experts." + std::to_string(e) + ".";
        v.push_back({ep + "gate_proj.weight", 0, 2, I, H});
        v.push_back({ep + "up_proj.weight", 0, 2, I, H});
        v.push_back({ep + "down_proj.weight", 0, 2, H, I});
    }
    if (c.n_shared_experts > 0) {
        const int64_t si = c.n_shared_experts * I;
        v.push_back({p + "mlp.shared_experts.gate_proj.weight", 0, 1, si, H});
        v.push_back({p + "mlp.shared_experts.up_proj.weight", 0, 1, si, H});
        v.push_back({p + "mlp.shared_experts.down_proj.weight", 0, 1, H, si});
    }
}

// Every tensor the config needs, with its shape (the names load_model_with
// reads, loader.rs:67-229).
void model_tensor_list(const ut_model_config &c, std::vector<SynthItem> &items) {
    const int64_t H = c.hidden_size, L = c.num_hidden_layers;
    items.push_back({"model.embed_tokens.weight", 0, 1, c.vocab_size, H});
    for (int64_t li = 0; li < L; li++) synth_layer_list(c, li, li < c.first_k_dense_replace, items);
    items.push_back({"model.norm.weight", 1, 0, H, 1});
    items.push_back({"lm_head.weight", 0, 1, c.vocab_size, H});
    if (c.mtp) {
        const std::string p = "model.layers." + std::to_string(L) + ".";
        synth_layer_list(c, L, false, items);
        items.push_back({p + "enorm.weight", 1, 0, H, 1});
        items.push_back({p + "hnorm.weight", 1, 0, H, 1});
        items.push_back({p + "eh_proj.weight", 0, 1, H, 2 * H});
        items.push_back({p + "shared_head.norm.weight", 1, 0, H, 1});
        items.push_back({p + "shared_head.head.weight", 0, 1, c.vocab_size, H});
    }
}

// Rows of an int8 embedding rescaled to unit RMS: scale[r] =
// 1 / sqrt(mean(code^2)) over the row's codes (the integer sum is exact).
__global__ __launch_bounds__(256) void k_unit_rms_scales(const int8_t *__restrict__ q, int64_t K,
                                                         float *__restrict__ scales) {
    __shared__ int64_t red[4];
    const int64_t r = blockIdx.x;
    int64_t acc = 0;
    for (int64_t i = threadIdx.x; i < K; i += 256) {
        const int v = q[r * K + i];
        acc += v * v;
    }
    for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        const int64_t t = red[0] + red[1] + red[2] + red[3];
        scales[r] = t > 0 ? 1.0f / sqrtf((float)((double)t / (double)K)) : 1.0f;
    }
}

// int8 [H, 2H] = [I | 0]: code 127 on the left block's diagonal.
__global__ void k_eye_left_i8(int8_t *__restrict__ q, int64_t H) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < H * 2 * H;
         i += (int64_t)gridDim.x * blockDim.x)
        q[i] = (i / (2 * H)) == (i % (2 * H)) ? (int8_t)127 : (int8_t)0;
}

__global__ void k_fill_f32(float *__restrict__ p, int64_t n, float v) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

// flags & UT_SYNTH_MTP_RESTATES: the construction of ut_model_synthesize_ex
// (the MTP module restates the first MoE layer; the other layers' residual
// writes damped by 2^-10; unit-RMS embedding rows; eh_proj = [I | 0]).
int32_t synthesize_all(ut_model *m, uint64_t seed, float std, int expert_fmt, int dense_fmt,
                       int flags = 0) {
    const ut_model_config &c = m->c;
    ut_ctx *ctx = m->ctx;
    std::vector<SynthItem> items;
    model_tensor_list(c, items);
    const bool restate = (flags & UT_SYNTH_MTP_RESTATES) != 0;
    const int64_t src_layer = c.first_k_dense_replace;  // the MoE layer the MTP module restates
    const std::string mtp_pre = "model.layers." + std::to_string(c.num_hidden_layers) + ".";
    const std::string src_pre = "model.layers." + std::to_string(src_layer) + ".";
    // the fills' keys by tensor name: a restating MTP tensor reuses its
    // source's keys, so the generator writes the same bytes
    std::unordered_map<std::string, std::pair<uint64_t, uint64_t>> keys;
    auto source_of = [&](const std::string &name) -> std::string {
        if (!restate) return std::string();
        if (name == mtp_pre + "shared_head.norm.weight") return "model.norm.weight";
        if (name == mtp_pre + "shared_head.head.weight") return "lm_head.weight";
        if (name.compare(0, mtp_pre.size(), mtp_pre) != 0) return std::string();
        const std::string rest = name.substr(mtp_pre.size());
        if (rest == "enorm.weight" || rest == "hnorm.weight" || rest == "eh_proj.weight")
            return std::string();
        return src_pre + rest;
    };
    // a residual write of a layer other than the restated one (o_proj, and
    // the down projections of the dense FFN, routed and shared experts)
    auto damped = [&](const std::string &name) -> bool {
        if (!restate || name.compare(0, 13, "model.layers.") != 0) return false;
        if (name.compare(0, src_pre.size(), src_pre) == 0 ||
            name.compare(0, mtp_pre.size(), mtp_pre) == 0)
            return false;
        const size_t n = name.size();
        auto ends = [&](const char *t) {
            const size_t k = strlen(t);
            return n >= k && name.compare(n - k, k, t) == 0;
        };
        return ends("self_attn.o_proj.weight") || ends("down_proj.weight");
    };
    constexpr float kDamp = 1.0f / 1024.0f;
    // one arena for everything, 256-byte aligned pieces
    auto al = [](int64_t b) { return (b + 255) & ~int64_t(255); };
    int64_t total = 0;
    for (auto &it : items) {
        if (m->store && it.cls == 2) continue;  // routed experts live in the store
        if (it.kind != 0) { total += al(it.d0 * 4); continue; }
        int fmt = it.cls == 0 ? UT_FMT_F32 : it.cls == 1 ? dense_fmt : expert_fmt;
        total += al(payload_bytes(fmt, it.d0, it.d1)) + (fmt == UT_FMT_F32 ? 0 : al(it.d0 * 4));
    }
    void *arena = nullptr;
    UT_TRY(dev_alloc(m, (size_t)total, &arena));
    char *p = (char *)arena;
    uint64_t idx = 0;
    uint64_t forced = 0;  // nonzero: the key of the next fill (a restated tensor's)
    uint64_t last_key = 0;
    auto fill = [&](void *dst, int64_t n, int kind, float a, float b) -> int32_t {
        const uint64_t key = forced ? forced : mix_host(seed, idx);
        idx++;
        forced = 0;
        last_key = key;
        int64_t blocks = (n + 255) / 256;
        if (blocks > 16384) blocks = 16384;
        hipLaunchKernelGGL(k_synth, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, dst, n,
                           kind, key, a, b);
        return launch_check(ctx, "k_synth");
    };
    auto grid = [](int64_t n) { return (unsigned)std::min<int64_t>((n + 255) / 256, 16384); };
    for (auto &it : items) {
        if (m->store && it.cls == 2) continue;
        DevTensor t;
        t.d0 = it.d0;
        t.d1 = it.d1;
        const std::string src = source_of(it.name);
        const auto ks = src.empty() ? keys.end() : keys.find(src);
        if (!src.empty() && ks == keys.end()) {
            set_error(ctx, "synthesize: %s has no source %s", it.name.c_str(), src.c_str());
            return UT_ERR_STATE;
        }
        if (it.kind != 0) {
            if (restate && it.name == mtp_pre + "enorm.weight") {
                hipLaunchKernelGGL(k_fill_f32, dim3(grid(it.d0)), dim3(256), 0, ctx->stream,
                                   (float *)p, it.d0, 1.0f);
                UT_TRY(launch_check(ctx, "k_fill_f32"));
                idx++;
            } else {
                if (ks != keys.end()) forced = ks->second.first;
                UT_TRY(fill(p, it.d0, it.kind == 1 ? 4 : 5, 0.0f, 0.0f));
            }
            keys[it.name] = {last_key, 0};
            t.vec = (float *)p;
            p += al(it.d0 * 4);
        } else {
            const int fmt = it.cls == 0 ? UT_FMT_F32 : it.cls == 1 ? dense_fmt : expert_fmt;
            ut_qtensor *q = new (std::nothrow) ut_qtensor();
            if (!q) return UT_ERR_OOM;
            q->fmt = fmt;
            q->out_dim = it.d0;
            q->in_dim = it.d1;
            q->row_bytes = payload_bytes(fmt, 1, it.d1);
            q->owns = false;
            q->device = m->device;
            q->payload = p;
            const int64_t pb = payload_bytes(fmt, it.d0, it.d1);
            const bool eye = restate && it.name == mtp_pre + "eh_proj.weight" && fmt == UT_FMT_INT8;
            const bool unit_rows = restate && it.name == "model.embed_tokens.weight" &&
                                   fmt == UT_FMT_INT8;
            uint64_t pkey = 0;
            if (ks != keys.end()) forced = ks->second.first;
            if (eye) {
                hipLaunchKernelGGL(k_eye_left_i8, dim3(grid(pb)), dim3(256), 0, ctx->stream,
                                   (int8_t *)p, it.d0);
                UT_TRY(launch_check(ctx, "k_eye_left_i8"));
                idx++;
            } else if (fmt == UT_FMT_F32) {
                UT_TRY(fill(p, it.d0 * it.d1, 3, std, 1.0f));
                pkey = last_key;
            } else {
                UT_TRY(fill(p, pb, fmt == UT_FMT_INT4 ? 0 : 1, 0.0f, 0.0f));
                pkey = last_key;
            }
            char *payload = p;
            p += al(pb);
            uint64_t skey = 0;
            if (fmt != UT_FMT_F32) {
                q->scales = (float *)p;
                if (eye) {
                    hipLaunchKernelGGL(k_fill_f32, dim3(grid(it.d0)), dim3(256), 0, ctx->stream,
                                       (float *)p, it.d0, 1.0f / 127.0f);
                    UT_TRY(launch_check(ctx, "k_fill_f32"));
                    idx++;
                } else if (unit_rows) {
                    hipLaunchKernelGGL(k_unit_rms_scales, dim3((unsigned)it.d0), dim3(256), 0,
                                       ctx->stream, (const int8_t *)payload, it.d1, (float *)p);
                    UT_TRY(launch_check(ctx, "k_unit_rms_scales"));
                    idx++;
                } else {
                    if (ks != keys.end()) forced = ks->second.second;
                    UT_TRY(fill(p, it.d0, 2, damped(it.name) ? std * kDamp : std,
                                fmt == UT_FMT_INT4 ? 7.0f : 127.0f));
                    skey = last_key;
                }
                p += al(it.d0 * 4);
            }
            keys[it.name] = {pkey, skey};
            t.qt = q;
        }
        m->tensors.emplace(it.name, t);
    }
    UT_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return UT_OK;
}

// ----------------------------------------------------- generation loops ---
// The emit rule shared by undertow_core::generate (core/model.rs:139-166)
// and the speculative loops (mtp.rs:194-257, 263-314): every emitted token
// goes to out and to on_token, and the stream ends after a stop token (the
// model's stop ids or the call's extra ids; the stop token is emitted and
// counted), when on_token returns 0, or at max_new tokens.
struct Emit {
    const ut_model *m;
    const int32_t *extra;
    int64_t n_extra;
    ut_token_fn on_token;
    void *user;
    int32_t *out;
    int64_t max_new;
    int64_t produced = 0;

    bool is_stop(int32_t tok) const {
        for (int32_t id : m->stop_ids)
            if (id == tok) return true;
        for (int64_t i = 0; i < n_extra; i++)
            if (extra[i] == tok) return true;
        return false;
    }
    // emits tok; true when the stream ends with it
    bool push(int32_t tok) {
        out[produced++] = tok;
        const bool keep = on_token ? on_token(user, tok) != 0 : true;
        return is_stop(tok) || !keep || produced >= max_new;
    }
};

// Greedy generation on a fresh session.  Each step is fed the previous
// step's argmax on the device, and the next step is queued before the host
// waits for the current token (a step queued past the stream's end is
// discarded with the session).
// Whether device-fed steps of this session may run from captured graphs:
// asked for, not given up on, every launch of the step on the device (no
// expert tier: it reads the routing back each layer), no kernel timing (its
// events), and one eager step of the same shape run first (eager_steps:
// host-side one-time set-up, such as occupancy queries and working-memory
// growth, happens there).
bool graph_ok(const ut_session *s, int64_t eager_steps) {
    const ut_model *m = s->m;
    return m->graphs && !s->graph_failed && !m->store && !s->ctx->timing && !fast8(s) &&
           eager_steps >= 1;
}

// Captures the launches of body() (a step of the session) into *exec.  The
// capture pass runs the host side of the step (so the session's positions
// advance as if it ran); every position-dependent launch reads the device
// word s->dpos, and attention grids are sized for the capacity.  The graph must hold kernel launches
// only.  The null stream cannot be captured: then the launches are captured
// on the context's own stream (capturing runs nothing) and the graph is
// launched on the context's stream.  On failure the host positions are
// restored and UT_ERR_STATE returned (the caller runs the step eagerly).
template <typename Body>
int32_t capture_body(ut_session *s, Body body, hipGraphExec_t *exec) {
    ut_model *m = s->m;
    ut_ctx *ctx = s->ctx;
    const hipStream_t run_stream = ctx->stream;
    ctx->stream = run_stream ? run_stream : ctx->own_stream;
    const int64_t pos0 = s->pos, mtp_len0 = s->mtp_kv.len;
    std::vector<int64_t> lens;
    for (auto &kv : s->kv) lens.push_back(kv.len);
    ctx->step_pos = s->dpos;
    ctx->step_pos_host = pos0;
    ctx->step_cap = s->cap;
    hipGraph_t graph = nullptr;
    int32_t rc = UT_OK;
    if (hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal) != hipSuccess) {
        rc = UT_ERR_STATE;
    } else {
        rc = body();
        if (hipStreamEndCapture(ctx->stream, &graph) != hipSuccess) rc = UT_ERR_STATE;
    }
    ctx->step_pos = nullptr;
    ctx->stream = run_stream;
    (void)hipGetLastError();
    if (rc == UT_OK && graph) {
        size_t nn = 0;
        if (hipGraphGetNodes(graph, nullptr, &nn) != hipSuccess) rc = UT_ERR_STATE;
        std::vector<hipGraphNode_t> nodes(nn);
        if (rc == UT_OK && nn && hipGraphGetNodes(graph, nodes.data(), &nn) != hipSuccess)
            rc = UT_ERR_STATE;
        for (size_t i = 0; rc == UT_OK && i < nn; i++) {
            hipGraphNodeType t;
            if (hipGraphNodeGetType(nodes[i], &t) != hipSuccess || t != hipGraphNodeTypeKernel)
                rc = UT_ERR_STATE;
        }
        if (rc == UT_OK && hipGraphInstantiate(exec, graph, nullptr, nullptr, 0) != hipSuccess) {
            *exec = nullptr;
            rc = UT_ERR_STATE;
        }
    } else if (rc == UT_OK) {
        rc = UT_ERR_STATE;
    }
    if (graph) (void)hipGraphDestroy(graph);
    (void)hipGetLastError();
    if (rc != UT_OK) {
        s->pos = pos0;
        for (size_t i = 0; i < lens.size(); i++) s->kv[i].len = lens[i];
        s->mtp_kv.len = mtp_len0;
        return UT_ERR_STATE;
    }
    return UT_OK;
}

int32_t capture_rows(ut_session *s, int64_t rows, const int32_t *ids_dev, hipGraphExec_t *exec) {
    return capture_body(s, [&]() -> int32_t {
        UT_TRY(prefill_dev(s, nullptr, rows, ids_dev));
        return launch_pos_add(s->ctx, s->dpos, rows);
    }, exec);
}

// One device-fed step of `rows` rows (ids at ids_dev): replayed from the
// graph *g when the session allows it (captured on first use), else
// launched eagerly.  eager_steps counts the steps of this shape.
int32_t graph_step(ut_session *s, int64_t rows, const int32_t *ids_dev, hipGraphExec_t *g,
                   int64_t *eager_steps) {
    ut_model *m = s->m;
    ut_ctx *ctx = s->ctx;
    if (!graph_ok(s, *eager_steps)) {
        const int32_t rc = prefill_dev(s, nullptr, rows, ids_dev);
        if (rc == UT_OK) (*eager_steps)++;
        return rc;
    }
    if (s->pos + rows > s->cap) {
        set_error(ctx, "context overflow: %lld + %lld > %lld", (long long)s->pos,
                  (long long)rows, (long long)s->cap);
        return UT_ERR_CONTEXT_OVERFLOW;
    }
    // the device position word must hold this step's position
    if (s->dpos_host != s->pos) {
        UT_TRY(launch_pos_set(ctx, s->dpos, s->pos));
        s->dpos_host = s->pos;
    }
    if (!*g) {
        if (capture_rows(s, rows, ids_dev, g) != UT_OK) {
            s->graph_failed = true;
            m->graph_failures++;
            return graph_step(s, rows, ids_dev, g, eager_steps);
        }
        m->graph_captures++;
        // the capture pass advanced the host positions; now run the step
    } else {
        s->pos += rows;
        for (auto &kv : s->kv) kv.len += rows;
    }
    UT_CHECK_HIP(ctx, hipGraphLaunch(*g, ctx->stream));
    m->graph_replays++;
    s->dpos_host += rows;
    (*eager_steps)++;
    return UT_OK;
}

// One device-fed decode step (its token in ws.am[0]).
int32_t decode_step(ut_session *s) { return graph_step(s, 1, s->ws.am, &s->g1, &s->m1_steps); }

// The MTP verify step: `rows` rows fed from ws.vids.
int32_t verify_step(ut_session *s, int64_t rows) {
    if (s->gv && s->gv_rows != rows) {
        (void)hipGraphExecDestroy(s->gv);
        s->gv = nullptr;
        s->v_steps = 0;
    }
    s->gv_rows = rows;
    return graph_step(s, rows, s->ws.vids, &s->gv, &s->v_steps);
}

// The MTP head's feed after a verify that accepted `pending - 1` drafts
// (mtp.rs:84-121): the ids of positions fed..pos-1 gathered on the device
// from the verify's ids and argmax rows, the main model's hidden rows at
// those positions read at the device position word, then the MTP layer and
// head on them (the draft into ws.vids[1]).  Replayed from a graph per row
// count when the session allows it, like the verify step.
int32_t draft_feed(ut_session *s, int64_t pending) {
    ut_model *m = s->m;
    ut_ctx *ctx = s->ctx;
    const int64_t H = m->c.hidden_size, fed = s->mtp_fed;
    auto body = [&]() -> int32_t {
        Workspace &w = s->ws;
        UT_TRY(launch_feed_ids(ctx, w.ids, w.vids, w.am, (int)pending - 1));
        UT_TRY(launch_copy_rows_from(ctx, w.attn, s->hidden, H, fed, pending, H));
        return draft_rows_dev(s, nullptr, -1, w.attn, pending, 1, w.ids);
    };
    hipGraphExec_t *g = &s->gd[pending - 1];
    int64_t *steps = &s->d_steps[pending - 1];
    if (!graph_ok(s, *steps)) {
        UT_TRY(body());
        (*steps)++;
        return UT_OK;
    }
    // the device position word must hold the main position
    if (s->dpos_host != s->pos) {
        UT_TRY(launch_pos_set(ctx, s->dpos, s->pos));
        s->dpos_host = s->pos;
    }
    if (!*g) {
        if (capture_body(s, body, g) != UT_OK) {
            s->graph_failed = true;
            m->graph_failures++;
            return draft_feed(s, pending);
        }
        m->graph_captures++;
        // the capture pass advanced the host's MTP cache length; now run it
    } else {
        s->mtp_kv.len += pending;
    }
    UT_CHECK_HIP(ctx, hipGraphLaunch(*g, ctx->stream));
    m->graph_replays++;
    (*steps)++;
    return UT_OK;
}

int64_t gen_greedy(ut_model *m, const int32_t *prompt, int64_t n, Emit &em) {
    ut_session *s = nullptr;
    UT_TRY(ut_session_create(m, 0, &s));
    std::vector<int32_t> am((size_t)(n > 0 ? n : 1));
    int32_t rc = prefill_dev(s, prompt, n);
    if (rc == UT_OK) rc = read_argmax(s, n, am.data());
    if (rc || em.max_new == 0) {
        ut_session_free(s);
        return rc;
    }
    int32_t tok = am[(size_t)n - 1];
    bool queued = false;  // a step whose output token is not read yet
    if (!em.push(tok)) {
        rc = prefill_dev(s, nullptr, 1, s->ws.am + (n - 1));
        if (rc == UT_OK) {
            s->tokens.push_back(tok);
            queued = true;
        } else if (rc == UT_ERR_CONTEXT_OVERFLOW) {
            rc = UT_OK;  // end of stream at the context end (core/model.rs:158-161)
        }
    }
    while (queued && rc == UT_OK) {
        rc = readback_enqueue(s, s->ws.am, 1, 0, RB_ERR_INLINE);
        if (rc) break;
        bool next_queued = false;
        if (em.produced + 1 < em.max_new) {
            // fed from ws.am[0], which this step overwrites only after reading it
            const int32_t r2 = decode_step(s);
            if (r2 == UT_OK) next_queued = true;
            else if (r2 != UT_ERR_CONTEXT_OVERFLOW) { rc = r2; break; }
        }
        rc = readback_wait(s, 1, &tok);
        if (rc) break;
        if (em.push(tok)) break;
        if (next_queued) s->tokens.push_back(tok);  // the id the queued step was fed
        queued = next_queued;
    }
    ut_session_free(s);
    return rc ? rc : em.produced;
}

// speculative_loop (mtp.rs:263-314) at depth 1..3.  Drafts come from the
// native MTP head (draft_fn == nullptr: draft_logits, mtp.rs:74-133, chained
// on its own output row for depth > 1) or from the caller's draft_fn.  One
// verify prefill of [next, d1..dk]; the longest prefix of drafts equal to
// the verify argmax rows is accepted; the main KV rolls back to the last
// verified position.
int64_t gen_spec(ut_model *m, const int32_t *prompt, int64_t n, int32_t depth, ut_draft_fn draft_fn,
                 void *draft_user, Emit &em, int64_t *drafted, int64_t *accepted) {
    ut_ctx *ctx = m->ctx;
    const int64_t H = m->c.hidden_size, V = m->c.vocab_size;
    ut_session *s = nullptr;
    UT_TRY(ut_session_create(m, 0, &s));
    std::vector<int32_t> am((size_t)(n > depth + 1 ? n : depth + 1));
    int32_t rc = prefill_dev(s, prompt, n);
    if (rc == UT_OK) rc = read_argmax(s, n, am.data());
    if (rc || em.max_new == 0) {
        ut_session_free(s);
        return rc;
    }
    int32_t next = am[(size_t)n - 1];
    int64_t nd = 0, na = 0;
    bool verified = false;  // a verify ran in this loop (its ids and argmax rows are on the device)
    std::vector<int32_t> toks, drafts((size_t)depth), vid((size_t)depth + 1);
    for (;;) {
        if (em.push(next)) break;
        const int64_t pos_before = s->pos;
        if (draft_fn) {
            // draft_fn(&session, next) (mtp.rs:263-314): the consumed tokens
            // and the emitted, not yet consumed `next`
            const int32_t r = draft_fn(draft_user, s->tokens.data(), (int64_t)s->tokens.size(),
                                       next, depth, drafts.data());
            if (r < 0) {
                set_error(ctx, "draft callback returned %d", r);
                rc = r;
                break;
            }
            for (int32_t d : drafts)
                if (d < 0 || d >= V) {
                    set_error(ctx, "draft id %d out of vocab (%lld)", d, (long long)V);
                    rc = UT_ERR_BAD_TOKEN;
                }
            if (rc) break;
            vid[0] = next;
            std::copy(drafts.begin(), drafts.end(), vid.begin() + 1);
            // the workspace holds at least four rows; vids must not move
            rc = ws_reserve(s, depth + 1);
            if (rc == UT_OK) rc = upload_slot(s, s->ws.vids, vid.data(), depth + 1, kPinIds - 8);
            if (rc) break;
        } else {
            // ---- draft: feed verified positions fed..pos-1 (mtp.rs:84-121);
            // after a verify their ids are the accepted drafts and `next`,
            // which the device holds (draft_feed), else they come from the host
            const int64_t pos = s->pos, fed = s->mtp_fed, pending = pos - fed;
            if (verified && pending >= 1 && pending <= depth + 1) {
                rc = draft_feed(s, pending);
            } else {
                toks.clear();
                for (int64_t i = fed; i < pos; i++)
                    toks.push_back(i + 1 < pos ? s->tokens[(size_t)i + 1] : next);
                rc = draft_rows_dev(s, toks.data(), -1, s->hidden + fed * H, pending, 1);
            }
            if (rc) break;
            s->mtp_fed = pos;
            // ---- chained drafts (depth > 1): MTP layer on its own last output row
            for (int32_t j = 1; j < depth && rc == UT_OK; j++) {
                // the MTP layer's output row for the last fed position is in
                // ws.x: the draft's first launch reads it (into its own input
                // rows) before anything of the draft writes ws.x
                const int64_t last = (j == 1 ? pending : 1) - 1;
                rc = draft_rows_dev(s, nullptr, j, s->ws.x + last * H, 1, 1 + j);
            }
            s->mtp_kv.len = s->mtp_fed;  // speculative MTP rows are never kept
            if (rc) break;
            rc = upload_slot(s, s->ws.vids, &next, 1, kPinIds - 8);
            if (rc) break;
        }
        nd += depth;
        // ---- verify [next, d1..dk] in one prefill, ids assembled on the device
        rc = verify_step(s, depth + 1);
        if (rc == UT_ERR_CONTEXT_OVERFLOW) {
            // no room for the verify rows: end the stream cleanly (mtp.rs:283-289;
            // the draft stays counted, as stats.drafted was bumped before)
            rc = UT_OK;
            break;
        }
        if (rc) break;
        // the verify's argmax rows, the flag and (after them, at depth + 2)
        // its drafts in one copy
        rc = readback_enqueue(s, s->ws.am, depth + 1, 0, RB_ERR_INLINE, draft_fn ? 0 : depth);
        if (rc == UT_OK) rc = readback_wait(s, depth + 1, am.data(), 0);
        if (rc) break;
        verified = true;
        if (!draft_fn) memcpy(drafts.data(), s->pin + kPinIds + depth + 2, (size_t)depth * 4);
        s->tokens.push_back(next);
        s->tokens.insert(s->tokens.end(), drafts.begin(), drafts.end());
        int64_t a = 0;
        bool end = false;
        while (a < depth && am[(size_t)a] == drafts[(size_t)a]) {
            a++;
            na++;
            if (em.push(drafts[(size_t)a - 1])) { end = true; break; }
        }
        if (end) break;
        next = am[(size_t)a];
        if (a < depth) truncate_session(s, pos_before + 1 + a);
    }
    if (drafted) *drafted = nd;
    if (accepted) *accepted = na;
    ut_session_free(s);
    return rc ? rc : em.produced;
}

}  // namespace

// ------------------------------------------------------- shard loader ---
// Host->device streaming through two pinned staging buffers: pread fills
// one while the copy engine drains the other (hipMemcpyAsync on the
// context's stream, an event per buffer marks when it may be refilled).
struct Stager {
    ut_ctx *ctx = nullptr;
    static constexpr size_t kChunk = size_t(64) << 20;
    void *pin[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    bool pending[2] = {false, false};
    int next = 0;
    uint64_t bytes_read = 0;
    std::vector<uint16_t> halves;

    int32_t init(ut_ctx *c) {
        ctx = c;
        for (int i = 0; i < 2; i++) {
            if (hipHostMalloc(&pin[i], kChunk, hipHostMallocDefault) != hipSuccess ||
                hipEventCreateWithFlags(&done[i], hipEventDisableTiming) != hipSuccess) {
                (void)hipGetLastError();
                set_error(ctx, "pinned staging allocation failed");
                return UT_ERR_OOM;
            }
        }
        return UT_OK;
    }
    ~Stager() {
        for (int i = 0; i < 2; i++) {
            if (pending[i]) (void)hipEventSynchronize(done[i]);
            if (pin[i]) (void)hipHostFree(pin[i]);
            if (done[i]) (void)hipEventDestroy(done[i]);
        }
    }
    int32_t take(void **buf) {
        const int b = next;
        next ^= 1;
        if (pending[b]) UT_CHECK_HIP(ctx, hipEventSynchronize(done[b]));
        pending[b] = false;
        *buf = pin[b];
        return b;
    }
    int32_t send(int b, void *dst, size_t n) {
        UT_CHECK_HIP(ctx, hipMemcpyAsync(dst, pin[b], n, hipMemcpyHostToDevice, ctx->stream));
        UT_CHECK_HIP(ctx, hipEventRecord(done[b], ctx->stream));
        pending[b] = true;
        return UT_OK;
    }
    // n bytes at offset of a shard to dst (device)
    int32_t raw(const st::Shard &sh, uint64_t offset, uint64_t n, char *dst) {
        for (uint64_t pos = 0; pos < n;) {
            const size_t len = (size_t)std::min<uint64_t>(kChunk, n - pos);
            void *buf = nullptr;
            int b = take(&buf);
            if (b < 0) return b;
            std::string err;
            if (!st::read_at(sh, buf, len, offset + pos, err)) {
                set_error(ctx, "%s", err.c_str());
                return UT_ERR_IO;
            }
            bytes_read += len;
            UT_TRY(send(b, dst + pos, len));
            pos += len;
        }
        return UT_OK;
    }
    // count 16-bit floats (bf16 or f16) at offset, widened exactly to f32 at dst
    int32_t widen(const st::Shard &sh, uint64_t offset, uint64_t count, bool bf16, float *dst) {
        const uint64_t per = kChunk / 4;
        halves.resize((size_t)std::min<uint64_t>(per, count));
        for (uint64_t pos = 0; pos < count;) {
            const uint64_t cnt = std::min<uint64_t>(per, count - pos);
            std::string err;
            if (!st::read_at(sh, halves.data(), cnt * 2, offset + pos * 2, err)) {
                set_error(ctx, "%s", err.c_str());
                return UT_ERR_IO;
            }
            bytes_read += cnt * 2;
            void *buf = nullptr;
            int b = take(&buf);
            if (b < 0) return b;
            st::widen_halves(halves.data(), cnt, bf16, (uint32_t *)buf);
            UT_TRY(send(b, dst + pos, (size_t)cnt * 4));
            pos += cnt;
        }
        return UT_OK;
    }
};

// read_qtensor (undertow-io/src/reader.rs:403-444) and the vector reads of
// load_model_with (loader.rs:67-229) for every tensor the config needs,
// streamed into one device arena.  skip_experts: leave the routed experts
// out (an expert store serves them).
int32_t load_dir_all(ut_model *m, const char *dir, bool skip_experts, int64_t *bytes_read) {
    ut_ctx *ctx = m->ctx;
    st::Index idx;
    std::string err;
    if (!st::open_dir(dir, idx, err)) {
        set_error(ctx, "%s", err.c_str());
        return err.find("No such file") != std::string::npos ||
                       err.find("Permission denied") != std::string::npos
                   ? UT_ERR_IO
                   : UT_ERR_FORMAT;
    }
    std::vector<SynthItem> items;
    model_tensor_list(m->c, items);
    struct Plan {
        const SynthItem *it;
        const st::Entry *data, *scales;
        int fmt;
        int64_t pb;
    };
    std::vector<Plan> plan;
    auto al = [](int64_t b) { return (b + 255) & ~int64_t(255); };
    int64_t total = 0;
    for (auto &it : items) {
        if (skip_experts && it.cls == 2) continue;
        const st::Entry *e = idx.find(it.name);
        if (!e) {
            set_error(ctx, "tensor not found: %s", it.name.c_str());
            return UT_ERR_NOT_FOUND;
        }
        Plan pl{&it, e, nullptr, UT_FMT_F32, 0};
        const bool floaty = e->dtype == st::ST_F32 || e->dtype == st::ST_BF16 || e->dtype == st::ST_F16;
        if (it.kind != 0) {
            if (!floaty || e->shape.size() != 1 || e->shape[0] != it.d0) {
                set_error(ctx, "shape mismatch for %s: expected [%lld]", it.name.c_str(), (long long)it.d0);
                return UT_ERR_SHAPE;
            }
            pl.pb = it.d0 * 4;
            total += al(pl.pb);
        } else if ((pl.scales = idx.find(it.name + ".scales"))) {
            // read_qtensor (reader.rs:410-430): the payload is read raw
            // whatever its dtype and its format inferred from the byte count;
            // the scales are read as f32 (F32, or BF16 / F16 widened exactly)
            const st::Entry *sc = pl.scales;
            const bool sc_floaty =
                sc->dtype == st::ST_F32 || sc->dtype == st::ST_BF16 || sc->dtype == st::ST_F16;
            if (!sc_floaty) {
                set_error(ctx, "%s.scales: cannot convert the tensor to f32", it.name.c_str());
                return UT_ERR_FORMAT;
            }
            if (sc->shape.size() != 1 || sc->shape[0] != it.d0) {
                set_error(ctx, "shape mismatch for %s.scales: expected [%lld]", it.name.c_str(),
                          (long long)it.d0);
                return UT_ERR_SHAPE;
            }
            if ((int64_t)e->nbytes == payload_bytes(UT_FMT_INT8, it.d0, it.d1)) pl.fmt = UT_FMT_INT8;
            else if ((int64_t)e->nbytes == payload_bytes(UT_FMT_INT4, it.d0, it.d1)) pl.fmt = UT_FMT_INT4;
            else {
                set_error(ctx, "%s: payload of %llu bytes matches neither int8 nor int4 for [%lld, %lld]",
                          it.name.c_str(), (unsigned long long)e->nbytes, (long long)it.d0,
                          (long long)it.d1);
                return UT_ERR_FORMAT;
            }
            pl.pb = (int64_t)e->nbytes;
            total += al(pl.pb) + al(it.d0 * 4);
        } else {
            if (!floaty || e->shape.size() != 2 || e->shape[0] != it.d0 || e->shape[1] != it.d1) {
                set_error(ctx, "shape mismatch for %s: expected [%lld, %lld]", it.name.c_str(),
                          (long long)it.d0, (long long)it.d1);
                return UT_ERR_SHAPE;
            }
            pl.pb = it.d0 * it.d1 * 4;
            total += al(pl.pb);
        }
        plan.push_back(pl);
    }
    Stager sg;
    UT_TRY(sg.init(ctx));
    void *arena = nullptr;
    UT_TRY(dev_alloc(m, (size_t)total, &arena));
    char *p = (char *)arena;
    auto fill_f32 = [&](const st::Entry *e, float *dst) -> int32_t {
        const st::Shard &sh = idx.shards[(size_t)e->shard];
        if (e->dtype == st::ST_F32) return sg.raw(sh, e->offset, e->nbytes, (char *)dst);
        return sg.widen(sh, e->offset, e->nbytes / 2, e->dtype == st::ST_BF16, dst);
    };
    for (auto &pl : plan) {
        const SynthItem &it = *pl.it;
        DevTensor t;
        t.d0 = it.d0;
        t.d1 = it.d1;
        if (it.kind != 0) {
            UT_TRY(fill_f32(pl.data, (float *)p));
            t.vec = (float *)p;
            p += al(pl.pb);
        } else {
            ut_qtensor *q = new (std::nothrow) ut_qtensor();
            if (!q) return UT_ERR_OOM;
            q->fmt = pl.fmt;
            q->out_dim = it.d0;
            q->in_dim = it.d1;
            q->row_bytes = payload_bytes(pl.fmt, 1, it.d1);
            q->owns = false;
            q->device = m->device;
            q->payload = p;
            t.qt = q;
            auto prev = m->tensors.find(it.name);
            if (prev != m->tensors.end() && prev->second.qt) ut_qtensor_free(prev->second.qt);
            m->tensors[it.name] = t;
            if (pl.fmt == UT_FMT_F32) {
                UT_TRY(fill_f32(pl.data, (float *)p));
                p += al(pl.pb);
            } else {
                UT_TRY(sg.raw(idx.shards[(size_t)pl.data->shard], pl.data->offset, pl.data->nbytes, p));
                p += al(pl.pb);
                q->scales = (float *)p;
                UT_TRY(fill_f32(pl.scales, (float *)p));
                p += al(it.d0 * 4);
            }
            continue;
        }
        auto prev = m->tensors.find(it.name);
        if (prev != m->tensors.end() && prev->second.qt) ut_qtensor_free(prev->second.qt);
        m->tensors[it.name] = t;
    }
    UT_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (bytes_read) *bytes_read = (int64_t)sg.bytes_read;
    return UT_OK;
}

extern "C" {

int32_t ut_model_create(ut_ctx *ctx, const ut_model_config *cfg, ut_model **out) {
    if (!ctx || !cfg || !out) return UT_ERR_ARG;
    *out = nullptr;
    const ut_model_config &c = *cfg;
    // DeepseekConfig::validate essentials (config.rs:154-216)
    if (c.vocab_size <= 0 || c.hidden_size <= 0 || c.num_hidden_layers < 0 ||
        c.num_attention_heads <= 0 || c.kv_lora_rank <= 0 || c.kv_lora_rank % 4 != 0 ||
        c.qk_rope_head_dim <= 0 ||
        c.qk_rope_head_dim % 2 != 0 || c.qk_nope_head_dim <= 0 || c.v_head_dim <= 0 ||
        c.max_position_embeddings <= 0 || c.num_experts_per_tok <= 0 ||
        c.num_experts_per_tok > 64 || c.n_group < 0 || c.n_group > 64 ||
        (c.n_routed_experts > 0 && c.n_routed_experts > 4096) ||
        (c.first_k_dense_replace < c.num_hidden_layers && c.n_routed_experts <= 0)) {
        set_error(ctx, "invalid model config");
        return UT_ERR_ARG;
    }
    ut_model *m = new (std::nothrow) ut_model();
    if (!m) return UT_ERR_OOM;
    m->ctx = ctx;
    m->c = c;
    m->device = ctx->device;
    ctx_retain(ctx);
    *out = m;
    return UT_OK;
}

int32_t ut_model_set_tensor(ut_model *m, const char *name, int32_t fmt, const void *payload,
                            int64_t nbytes, const float *scales, int64_t d0, int64_t d1) {
    if (!m || !name || !payload || d0 <= 0 || d1 <= 0) {
        if (m) set_error(m->ctx, "ut_model_set_tensor: bad argument");
        return UT_ERR_ARG;
    }
    if (m->finalized) {
        set_error(m->ctx, "model already finalized");
        return UT_ERR_STATE;
    }
    DevTensor t;
    t.d0 = d0;
    t.d1 = d1;
    if (d1 == 1 && !scales && (fmt == UT_FMT_F32 || fmt == UT_FMT_INFER)) {
        if (nbytes != d0 * 4) {
            set_error(m->ctx, "%s: %lld bytes for a %lld-vector", name, (long long)nbytes, (long long)d0);
            return UT_ERR_FORMAT;
        }
        void *p = nullptr;
        UT_TRY(dev_alloc(m, (size_t)nbytes, &p));
        UT_CHECK_HIP(m->ctx, hipMemcpy(p, payload, (size_t)nbytes, hipMemcpyHostToDevice));
        t.vec = (float *)p;
    } else {
        ut_qtensor *q = nullptr;
        UT_TRY(ut_qtensor_upload(m->ctx, fmt, payload, nbytes, scales, scales ? d0 : 0, d0, d1, &q));
        m->device_bytes += ut_qtensor_nbytes(q);
        t.qt = q;
    }
    auto it = m->tensors.find(name);
    if (it != m->tensors.end()) {
        if (it->second.qt) ut_qtensor_free(it->second.qt);
        it->second = t;
    } else {
        m->tensors.emplace(name, t);
    }
    return UT_OK;
}

int32_t ut_model_load_dir(ut_model *m, const char *dir, int64_t *bytes_read) {
    if (!m || !dir) return UT_ERR_ARG;
    if (m->finalized || !m->tensors.empty()) {
        set_error(m->ctx, "ut_model_load_dir needs a fresh model");
        return UT_ERR_STATE;
    }
    UT_TRY(load_dir_all(m, dir, false, bytes_read));
    return ut_model_finalize(m);
}

}  // extern "C"

namespace {

int32_t make_store(ut_model *m, int expert_fmt, const ut_expert_store_config *cfg) {
    const ut_model_config &c = m->c;
    if (cfg->hbm_budget_bytes < 0 || (cfg->policy != 0 && cfg->policy != 1)) {
        set_error(m->ctx, "expert store: bad budget or policy");
        return UT_ERR_ARG;
    }
    if (c.n_routed_experts <= 0) {
        set_error(m->ctx, "expert store: the model has no routed experts");
        return UT_ERR_ARG;
    }
    m->store = new (std::nothrow) ut::ExpertStore();
    if (!m->store) return UT_ERR_OOM;
    m->store_prefetch = cfg->prefetch != 0;
    const int64_t layers = c.num_hidden_layers + (c.mtp ? 1 : 0);
    return m->store->init(m->ctx, layers, c.n_routed_experts, c.hidden_size,
                          c.moe_intermediate_size, expert_fmt, cfg->hbm_budget_bytes, cfg->policy,
                          4 * c.num_experts_per_tok);
}

int32_t need_store(const ut_model *m) {
    if (!m) return UT_ERR_ARG;
    if (!m->store) {
        set_error(m->ctx, "the model has no expert store (all experts resident)");
        return UT_ERR_STATE;
    }
    return UT_OK;
}

}  // namespace

extern "C" {

int32_t ut_model_load_dir_tiered(ut_model *m, const char *dir, const ut_expert_store_config *cfg,
                                 int64_t *bytes_read) {
    if (!m || !dir || !cfg) return UT_ERR_ARG;
    if (m->finalized || !m->tensors.empty() || m->store) {
        set_error(m->ctx, "ut_model_load_dir_tiered needs a fresh model");
        return UT_ERR_STATE;
    }
    // the experts' format from the first routed expert's payload size
    // (read_qtensor's inference, reader.rs:421-430)
    int fmt = UT_FMT_F32;
    {
        ut::st::Index idx;
        std::string err;
        if (!ut::st::open_dir(dir, idx, err)) {
            set_error(m->ctx, "%s", err.c_str());
            return err.find("No such file") != std::string::npos ? UT_ERR_IO : UT_ERR_FORMAT;
        }
        const int64_t L0 = m->c.first_k_dense_replace < m->c.num_hidden_layers
                               ? m->c.first_k_dense_replace : m->c.num_hidden_layers;
        const std::string n = "model.layers." + std::to_string(L0) + ".mlp.experts.0.gate_proj.weight";
        const ut::st::Entry *e = idx.find(n);
        if (!e) {
            set_error(m->ctx, "tensor not found: %s", n.c_str());
            return UT_ERR_NOT_FOUND;
        }
        const int64_t I = m->c.moe_intermediate_size, H = m->c.hidden_size;
        if (idx.find(n + ".scales"))
            fmt = (int64_t)e->nbytes == payload_bytes(UT_FMT_INT8, I, H) ? UT_FMT_INT8 : UT_FMT_INT4;
    }
    UT_TRY(make_store(m, fmt, cfg));
    UT_TRY(load_dir_all(m, dir, true, bytes_read));
    UT_TRY(ut_model_finalize(m));
    return m->store->attach_disk(dir);
}

int32_t ut_model_synthesize_tiered(ut_model *m, uint64_t seed, float init_std, int32_t expert_fmt,
                                   int32_t dense_fmt, const ut_expert_store_config *cfg,
                                   int64_t host_pool_experts) {
    if (!m || !cfg || host_pool_experts <= 0) return UT_ERR_ARG;
    if (m->finalized || !m->tensors.empty() || m->store) {
        set_error(m->ctx, "ut_model_synthesize_tiered needs a fresh model");
        return UT_ERR_STATE;
    }
    if ((expert_fmt != UT_FMT_INT4 && expert_fmt != UT_FMT_INT8) ||
        (dense_fmt != UT_FMT_INT4 && dense_fmt != UT_FMT_INT8)) {
        set_error(m->ctx, "synthesize: formats must be int4 or int8");
        return UT_ERR_ARG;
    }
    UT_TRY(make_store(m, expert_fmt, cfg));
    UT_TRY(synthesize_all(m, seed, init_std, expert_fmt, dense_fmt));
    UT_TRY(ut_model_finalize(m));
    return m->store->attach_host_pool(host_pool_experts, seed, init_std);
}

int32_t ut_model_pin_experts(ut_model *m, const int32_t *layer_expert, int64_t n,
                             int64_t budget_bytes, int64_t *pinned_bytes) {
    UT_TRY(need_store(m));
    if (n < 0 || (n > 0 && !layer_expert) || budget_bytes < 0) return UT_ERR_ARG;
    return m->store->pin(layer_expert, n, budget_bytes, pinned_bytes);
}

int32_t ut_model_store_stats(ut_model *m, ut_store_stats *out) {
    UT_TRY(need_store(m));
    if (!out) return UT_ERR_ARG;
    const ut::StoreStats &st = m->store->stats();
    out->hits = st.hits;
    out->misses = st.misses;
    out->bytes_read = st.bytes_read;
    out->evictions = st.evictions;
    out->prefetch_issued = st.prefetch_issued;
    out->prefetch_dropped = st.prefetch_dropped;
    out->bytes_used = st.bytes_used;
    out->budget_bytes = st.budget_bytes;
    out->pinned_experts = st.pinned;
    out->read_seconds = st.read_seconds;
    return UT_OK;
}

int32_t ut_model_expert_usage(ut_model *m, int64_t *counts, int64_t n) {
    UT_TRY(need_store(m));
    const std::vector<int64_t> &u = m->store->usage();
    if (!counts || n != (int64_t)u.size()) {
        set_error(m->ctx, "expert usage holds %lld counts", (long long)u.size());
        return UT_ERR_SHAPE;
    }
    std::copy(u.begin(), u.end(), counts);
    return UT_OK;
}

int32_t ut_model_finalize(ut_model *m) {
    if (!m) return UT_ERR_ARG;
    if (m->finalized) return UT_OK;
    ut_ctx *ctx = m->ctx;
    const ut_model_config &c = m->c;
    const int64_t H = c.hidden_size;
    UT_CHECK_HIP(ctx, hipSetDevice(m->device));
    UT_TRY(get_qt(m, "model.embed_tokens.weight", c.vocab_size, H, &m->embed));
    UT_TRY(get_qt(m, "lm_head.weight", c.vocab_size, H, &m->lm_head));
    UT_TRY(get_vec(m, "model.norm.weight", H, &m->final_norm));
    m->layers.assign((size_t)c.num_hidden_layers, LayerW());
    for (int64_t li = 0; li < c.num_hidden_layers; li++)
        UT_TRY(load_layer(m, li, li < c.first_k_dense_replace, &m->layers[li]));
    const std::string p = "model.layers." + std::to_string(c.num_hidden_layers) + ".";
    if (c.mtp && find(m, p + "eh_proj.weight")) {
        // MTP head (loader.rs:201-229): its layer is an MoE layer keyed at
        // index num_hidden_layers
        m->has_mtp = true;
        UT_TRY(get_qt(m, p + "eh_proj.weight", H, 2 * H, &m->eh_proj));
        UT_TRY(get_vec(m, p + "enorm.weight", H, &m->enorm));
        UT_TRY(get_vec(m, p + "hnorm.weight", H, &m->hnorm));
        UT_TRY(load_layer(m, c.num_hidden_layers, false, &m->mtp_layer));
        UT_TRY(get_vec(m, p + "shared_head.norm.weight", H, &m->mtp_norm));
        UT_TRY(get_qt(m, p + "shared_head.head.weight", c.vocab_size, H, &m->mtp_head));
    }
    // RoPE table with the host libm (attention.rs:110-113):
    // inv_j = theta^(-2j/dim), ang = pos*inv_j, (cos, sin)
    const int64_t rope = c.qk_rope_head_dim, half = rope / 2, P = c.max_position_embeddings;
    std::vector<float2> tab((size_t)(P * half));
    for (int64_t j = 0; j < half; j++) {
        const float inv = powf(c.rope_theta, -2.0f * (float)j / (float)rope);
        for (int64_t pos = 0; pos < P; pos++) {
            const float ang = (float)pos * inv;
            tab[(size_t)(pos * half + j)] = make_float2(cosf(ang), sinf(ang));
        }
    }
    void *tp = nullptr;
    UT_TRY(dev_alloc(m, tab.size() * sizeof(float2), &tp));
    UT_CHECK_HIP(ctx, hipMemcpy(tp, tab.data(), tab.size() * sizeof(float2), hipMemcpyHostToDevice));
    m->rope_table = (float2 *)tp;
    void *z = nullptr, *o = nullptr;
    UT_TRY(dev_alloc(m, 16, &z));
    UT_TRY(dev_alloc(m, 16, &o));
    const int32_t zs[4] = {0, 0, 0, 0};
    const float os[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    UT_CHECK_HIP(ctx, hipMemcpy(z, zs, 16, hipMemcpyHostToDevice));
    UT_CHECK_HIP(ctx, hipMemcpy(o, os, 16, hipMemcpyHostToDevice));
    m->zeros = (int32_t *)z;
    m->ones = (float *)o;
    // fixed plan of an MLP run as a one-expert block: count 1, slot 0 = expert 0
    void *pl = nullptr;
    UT_TRY(dev_alloc(m, 64, &pl));
    const int32_t plan_init[16] = {1, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    UT_CHECK_HIP(ctx, hipMemcpy(pl, plan_init, 64, hipMemcpyHostToDevice));
    m->mlp_plan.count = (int32_t *)pl;
    m->mlp_plan.uniq = (int32_t *)pl + 4;
    m->mlp_plan.choice_slot = (int32_t *)pl + 8;
    m->finalized = true;
    return UT_OK;
}

int64_t ut_model_device_bytes(const ut_model *m) { return m ? m->device_bytes : UT_ERR_ARG; }

void ut_model_free(ut_model *m) {
    if (!m || --m->refs > 0) return;  // live sessions keep the model
    (void)hipSetDevice(m->device);
    (void)hipStreamSynchronize(m->ctx->stream);
    for (auto &kv : m->tensors)
        if (kv.second.qt) ut_qtensor_free(kv.second.qt);
    for (void *p : m->device_allocs) (void)hipFree(p);
    delete m->store;
    ut_ctx *ctx = m->ctx;
    delete m;
    ctx_release(ctx);
}

int32_t ut_model_set_kv_budget(ut_model *m, int64_t kv_budget_bytes) {
    if (!m) return UT_ERR_ARG;
    if (kv_budget_bytes == 0) {
        set_error(m->ctx, "KV budget of 0 bytes");
        return UT_ERR_ARG;
    }
    m->kv_budget = kv_budget_bytes < 0 ? -1 : kv_budget_bytes;
    return UT_OK;
}

int64_t ut_model_max_context(const ut_model *m) {
    if (!m) return UT_ERR_ARG;
    const ut_model_config &c = m->c;
    if (m->kv_budget < 0) return c.max_position_embeddings;
    // loader.rs:311-325: per position the compressed latents of every main
    // layer, plus (with the MTP head) the saved hidden state and token id
    const int64_t per = c.num_hidden_layers * (c.kv_lora_rank + c.qk_rope_head_dim) * 4 +
                        (m->has_mtp ? c.hidden_size * 4 + 8 : 0);
    int64_t eff = m->kv_budget / (per > 0 ? per : 1);
    if (eff < 1) eff = 1;
    return eff < c.max_position_embeddings ? eff : c.max_position_embeddings;
}

int32_t ut_session_create(ut_model *m, int32_t path, ut_session **out) {
    return ut_session_create_on(m, nullptr, path, out);
}

int32_t ut_session_create_on(ut_model *m, ut_ctx *sctx, int32_t path, ut_session **out) {
    if (!m || !out) return UT_ERR_ARG;
    *out = nullptr;
    ut_ctx *ctx = sctx ? sctx : m->ctx;
    if (!m->finalized) {
        set_error(ctx, "model not finalized");
        return UT_ERR_STATE;
    }
    if (path < 0 || path > 2) {
        set_error(ctx, "bad attention path %d", path);
        return UT_ERR_ARG;
    }
    if (ctx != m->ctx) {
        if (ctx->device != m->device) {
            set_error(ctx, "session context on device %d, model on device %d", ctx->device,
                      m->device);
            return UT_ERR_ARG;
        }
        // the HBM tier's slots and tables change in the model's stream order
        if (m->store) {
            set_error(ctx, "sessions on another context need all routed experts resident");
            return UT_ERR_STATE;
        }
    }
    ut_session *s = new (std::nothrow) ut_session();
    if (!s) return UT_ERR_OOM;
    s->m = m;
    s->ctx = ctx;
    m->refs++;
    if (ctx != m->ctx) ctx_retain(ctx);
    s->path = path;
    s->cap = ut_model_max_context(m);
    const ut_model_config &c = m->c;
    const int64_t nl = c.num_hidden_layers + (m->has_mtp ? 1 : 0);
    const size_t per = (size_t)s->cap * (c.kv_lora_rank + c.qk_rope_head_dim) * 4;
    const size_t hid = m->has_mtp ? (size_t)s->cap * c.hidden_size * 4 : 0;
    if (hipMalloc(&s->kv_alloc, per * nl + hid + 512) != hipSuccess) {
        (void)hipGetLastError();
        set_error(m->ctx, "KV cache allocation failed");
        delete s;
        return UT_ERR_OOM;
    }
    char *p = (char *)s->kv_alloc;
    s->kv.resize((size_t)c.num_hidden_layers);
    // DeepSeek-V3-shaped attention keeps the cache in the MFMA kernel's
    // split bf16 form (the same bytes as the f32 cache)
    const bool split = mla_kc_ok(c.num_attention_heads, c.kv_lora_rank, c.qk_rope_head_dim, s->cap);
    auto carve = [&](KvCache &kv) {
        kv.latent = (float *)p;
        kv.krot = (float *)(p + (size_t)s->cap * c.kv_lora_rank * 4);
        kv.kc = split ? (__bf16 *)p : nullptr;
        kv.len = 0;
        p += per;
    };
    for (auto &kv : s->kv) carve(kv);
    if (m->has_mtp) {
        carve(s->mtp_kv);
        s->hidden = (float *)p;
        p += hid;
    }
    s->dpos = (int64_t *)((char *)s->kv_alloc + ((per * nl + hid + 255) & ~size_t(255)));
    if (hipHostMalloc((void **)&s->pin, (size_t)(kPinIds + kPinBack) * 4, hipHostMallocDefault) != hipSuccess ||
        hipEventCreateWithFlags(&s->ready, hipEventDisableTiming) != hipSuccess) {
        (void)hipGetLastError();
        set_error(m->ctx, "session staging allocation failed");
        ut_session_free(s);
        return UT_ERR_OOM;
    }
    int32_t rc = ws_reserve(s, 4);
    if (rc) {
        ut_session_free(s);
        return rc;
    }
    *out = s;
    return UT_OK;
}

void ut_session_free(ut_session *s) {
    if (!s) return;
    (void)hipSetDevice(s->m->device);
    (void)hipStreamSynchronize(s->ctx->stream);
    if (s->g1) (void)hipGraphExecDestroy(s->g1);
    if (s->gv) (void)hipGraphExecDestroy(s->gv);
    for (auto g : s->gd)
        if (g) (void)hipGraphExecDestroy(g);
    if (s->ws.base) (void)hipFree(s->ws.base);
    if (s->kv_alloc) (void)hipFree(s->kv_alloc);
    if (s->pin) (void)hipHostFree(s->pin);
    if (s->ready) (void)hipEventDestroy(s->ready);
    ut_model *m = s->m;
    ut_ctx *own = s->ctx != m->ctx ? s->ctx : nullptr;
    delete s;
    if (own) ctx_release(own);
    ut_model_free(m);  // drops the session's reference
}

int32_t ut_session_prefill(ut_session *s, const int32_t *ids, int64_t n, float *logits_host,
                           int32_t *argmax_host) {
    if (!s || (!ids && n > 0)) return UT_ERR_ARG;
    ut_ctx *ctx = s->ctx;
    UT_TRY(prefill_dev(s, ids, n));
    if (logits_host) {
        UT_CHECK_HIP(ctx, hipMemcpyAsync(logits_host, s->ws.logits,
                                         (size_t)n * s->m->c.vocab_size * 4,
                                         hipMemcpyDeviceToHost, ctx->stream));
    }
    std::vector<int32_t> am((size_t)n);
    UT_TRY(read_argmax(s, n, am.data()));
    if (argmax_host) memcpy(argmax_host, am.data(), (size_t)n * 4);
    return UT_OK;
}

int32_t ut_session_truncate(ut_session *s, int64_t len) {
    if (!s || len < 0) return UT_ERR_ARG;
    truncate_session(s, len);
    return UT_OK;
}

int64_t ut_session_position(const ut_session *s) { return s ? s->pos : UT_ERR_ARG; }

int32_t ut_model_set_stop_ids(ut_model *m, const int32_t *ids, int64_t n) {
    // DeepseekMoeModel::stop_ids (adapters/undertow-deepseek-moe/src/
    // loader.rs:304-309): the config's eos ids plus generation_config's
    if (!m || n < 0 || (n > 0 && !ids)) return UT_ERR_ARG;
    m->stop_ids.assign(ids, ids + n);
    return UT_OK;
}

int32_t ut_model_enable_graphs(ut_model *m, int32_t on) {
    if (!m) return UT_ERR_ARG;
    m->graphs = on != 0;
    return UT_OK;
}

int32_t ut_model_graph_stats(const ut_model *m, int64_t *captures, int64_t *replays,
                             int64_t *failures) {
    if (!m) return UT_ERR_ARG;
    if (captures) *captures = m->graph_captures;
    if (replays) *replays = m->graph_replays;
    if (failures) *failures = m->graph_failures;
    return UT_OK;
}

int64_t ut_generate(ut_model *m, const int32_t *prompt, int64_t n, int64_t max_new,
                    const int32_t *extra_stop_ids, int64_t n_extra, ut_token_fn on_token,
                    void *user, int32_t *out) {
    if (!m || !prompt || (max_new > 0 && !out) || max_new < 0 || n_extra < 0 ||
        (n_extra > 0 && !extra_stop_ids))
        return UT_ERR_ARG;
    Emit em{m, extra_stop_ids, n_extra, on_token, user, out, max_new};
    return gen_greedy(m, prompt, n, em);
}

int64_t ut_generate_greedy(ut_model *m, const int32_t *prompt, int64_t n, int64_t max_new,
                           int32_t *out) {
    return ut_generate(m, prompt, n, max_new, nullptr, 0, nullptr, nullptr, out);
}

int64_t ut_speculative_loop(ut_model *m, const int32_t *prompt, int64_t n, int64_t max_new,
                            int32_t depth, const int32_t *extra_stop_ids, int64_t n_extra,
                            ut_token_fn on_token, void *user, ut_draft_fn draft_fn,
                            void *draft_user, int32_t *out, int64_t *drafted, int64_t *accepted) {
    if (drafted) *drafted = 0;
    if (accepted) *accepted = 0;
    if (!m || !prompt || (max_new > 0 && !out) || max_new < 0 || n_extra < 0 ||
        (n_extra > 0 && !extra_stop_ids))
        return UT_ERR_ARG;
    if (depth < 1 || depth > 3) {
        set_error(m->ctx, "MTP depth %d outside 1..3", depth);
        return UT_ERR_ARG;
    }
    if (!draft_fn && !m->has_mtp) {
        set_error(m->ctx, "model has no MTP head; use plain generation");
        return UT_ERR_STATE;
    }
    Emit em{m, extra_stop_ids, n_extra, on_token, user, out, max_new};
    return gen_spec(m, prompt, n, depth, draft_fn, draft_user, em, drafted, accepted);
}

int64_t ut_generate_mtp(ut_model *m, const int32_t *prompt, int64_t n, int64_t max_new,
                        int32_t depth, int32_t *out, int64_t *drafted, int64_t *accepted) {
    return ut_speculative_loop(m, prompt, n, max_new, depth, nullptr, 0, nullptr, nullptr, nullptr,
                               nullptr, out, drafted, accepted);
}

int32_t ut_session_draft_logits(ut_session *s, int32_t next_token, float *logits_host,
                                int32_t *draft_host) {
    // draft_logits (mtp.rs:74-133) on the session's own MTP state: feeds
    // positions fed..pos-1 (t_next = the following consumed token, or
    // next_token for the last) and returns the head's logits for the last
    if (!s) return UT_ERR_ARG;
    ut_model *m = s->m;
    ut_ctx *ctx = s->ctx;
    const int64_t H = m->c.hidden_size, V = m->c.vocab_size;
    if (!m->has_mtp) {
        set_error(ctx, "model has no MTP head");
        return UT_ERR_STATE;
    }
    if (next_token < 0 || next_token >= V) {
        set_error(ctx, "token id %d out of vocab (%lld)", next_token, (long long)V);
        return UT_ERR_BAD_TOKEN;
    }
    const int64_t pos = s->pos, fed = s->mtp_fed;
    if (pos <= fed) {
        set_error(ctx, "draft with nothing pending (position %lld, fed %lld)", (long long)pos,
                  (long long)fed);
        return UT_ERR_STATE;
    }
    std::vector<int32_t> toks;
    for (int64_t i = fed; i < pos; i++) toks.push_back(i + 1 < pos ? s->tokens[(size_t)i + 1] : next_token);
    UT_TRY(draft_rows_dev(s, toks.data(), -1, s->hidden + fed * H, pos - fed, 1));
    s->mtp_fed = pos;
    if (logits_host)
        UT_CHECK_HIP(ctx, hipMemcpyAsync(logits_host, s->ws.logits, (size_t)V * 4,
                                         hipMemcpyDeviceToHost, ctx->stream));
    int32_t d = 0;
    UT_TRY(readback_enqueue(s, s->ws.vids + 1, 1));
    UT_TRY(readback_wait(s, 1, &d));
    if (draft_host) *draft_host = d;
    return UT_OK;
}

int32_t ut_model_synthesize(ut_model *m, uint64_t seed, float init_std, int32_t expert_fmt,
                            int32_t dense_fmt) {
    return ut_model_synthesize_ex(m, seed, init_std, expert_fmt, dense_fmt, 0);
}

int32_t ut_model_synthesize_ex(ut_model *m, uint64_t seed, float init_std, int32_t expert_fmt,
                               int32_t dense_fmt, int32_t flags) {
    if (!m) return UT_ERR_ARG;
    if (flags & ~UT_SYNTH_MTP_RESTATES) {
        set_error(m->ctx, "synthesize: unknown flags 0x%x", (unsigned)flags);
        return UT_ERR_ARG;
    }
    if ((flags & UT_SYNTH_MTP_RESTATES) &&
        (!m->c.mtp || dense_fmt != UT_FMT_INT8 ||
         m->c.first_k_dense_replace >= m->c.num_hidden_layers)) {
        set_error(m->ctx, "synthesize: a restating MTP module needs an MTP module, int8 dense "
                          "weights and a MoE layer");
        return UT_ERR_ARG;
    }
    if (m->finalized || !m->tensors.empty()) {
        set_error(m->ctx, "ut_model_synthesize needs a fresh model");
        return UT_ERR_STATE;
    }
    if ((expert_fmt != UT_FMT_INT4 && expert_fmt != UT_FMT_INT8) ||
        (dense_fmt != UT_FMT_INT4 && dense_fmt != UT_FMT_INT8)) {
        set_error(m->ctx, "synthesize: formats must be int4 or int8");
        return UT_ERR_ARG;
    }
    UT_TRY(synthesize_all(m, seed, init_std, expert_fmt, dense_fmt, flags));
    return ut_model_finalize(m);
}

}  // extern "C"
