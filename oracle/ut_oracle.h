/*
 * ut_oracle.h -- CPU restatement of the undertow reference's hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * path: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it.  The product library (undertow_amd, libundertow_hip.so) never
 * links or calls it.
 *
 * Every function restates a reference routine (Rust, mohitmishra786/undertow)
 * whose file:line is cited beside the declaration.  The reference cannot be
 * compiled here (no Rust toolchain), so this restatement is pinned instead by:
 *   - byte-exact regeneration of undertow-bench/fixtures/oracle-tiny/
 *     model.safetensors (sha256 in tests/golden),
 *   - the transformers golden reference.json of that fixture (teacher-forcing
 *     logits < 1e-3, argmax and greedy continuation exact),
 *   - the reference's unit known-answer tests, restated as data,
 *   - closed forms / brute force on small inputs.
 *
 * Numerical contract: scalar f32 in index order, compiled with
 * -ffp-contract=off (Rust never contracts a*b+c into an FMA), glibc libm for
 * expf/powf/sinf/cosf (the calls Rust's std makes on Linux).
 */
#ifndef UT_ORACLE_H
#define UT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* QuantFormat (undertow-quant/src/qtensor.rs:17-21). */
enum { UTO_F32 = 0, UTO_INT8 = 1, UTO_INT4 = 2 };

/* ---------------------------------------------------------------- RNG ---- */
/* Pcg32 + Irwin-Hall normal (undertow-bench/src/rng.rs:9-53). */
typedef struct { uint64_t state, inc; } uto_pcg32;
void     uto_pcg32_init(uto_pcg32 *r, uint64_t seed, uint64_t stream);
uint32_t uto_pcg32_next(uto_pcg32 *r);
float    uto_pcg32_uniform(uto_pcg32 *r);
float    uto_pcg32_normal(uto_pcg32 *r);
/* Fill n values; kind 0 = uniform, 1 = normal*std (normal_scaled). */
void     uto_pcg32_fill(uint64_t seed, uint64_t stream, int kind, float std,
                        float *out, int64_t n);

/* ------------------------------------------------------------- quant ----- */
/* unpack_i4 (undertow-quant/src/kernels.rs:10-19). */
int8_t uto_unpack_i4(const uint8_t *row, int64_t i);
/* QuantFormat::payload_bytes (qtensor.rs:43-49). */
int64_t uto_payload_bytes(int fmt, int64_t out_dim, int64_t in_dim);
/* QTensor::quantize (qtensor.rs:142-213).  Returns 0, or -1 on a non-finite
 * weight (the reference's Err).  payload: int8 codes or packed int4 rows. */
int uto_quantize(int fmt, const float *w, int64_t out_dim, int64_t in_dim,
                 void *payload, float *scales);
/* QTensor::dequantize = add_scaled_row(r, 1.0) into zeros (qtensor.rs:265-272,
 * 516-543): w = 0 + (1*scale)*q. */
void uto_dequantize(int fmt, const void *payload, const float *scales,
                    int64_t out_dim, int64_t in_dim, float *out);
/* Scalar kernels: kernels::matmul_i8/matmul_i4 (kernels.rs:21-81) and the f32
 * lib::matmul (undertow-quant/src/lib.rs:128-144); QTensor::matmul_scalar
 * (qtensor.rs:496-507).  out[s,o] = (sum_i x[s,i]*q[o,i]) * scale[o]. */
void uto_matmul(int fmt, const void *payload, const float *scales,
                int64_t out_dim, int64_t in_dim, const float *x, int64_t seq,
                float *out);
/* The opt-in fast-int8 path (undertow-quant/src/lib.rs:31-59): one
 * activation row quantised symmetrically to i8 with one scale
 * (quantize_activations: max = fold of max(|v|) from 0, which skips NaN;
 * scale = max/127, inv = 127/max, q = round(v*inv) half away from zero,
 * clamped to +-127, NaN -> 0; a zero row gives scale 0), then
 * avx512::matmul_i8_vnni (avx512.rs:221-242) / neon::matmul_i8_sdot
 * (neon.rs:139-184): out[s,o] = (acc as f32) * a_scale * scale[o] with acc
 * the exact integer dot of the i8 activations and the i8 codes. */
float uto_quantize_activations(const float *x, int64_t n, int8_t *out);
/* set_fast_int8 / fast_int8_enabled (lib.rs:35-43): while set, uto_matmul
 * on int8 weights is uto_matmul_fast_i8 (every int8 matmul of the model). */
void uto_set_fast_int8(int on);
int uto_fast_int8_enabled(void);
void uto_matmul_fast_i8(const int8_t *q, const float *scales, int64_t out_dim, int64_t in_dim,
                        const float *x, int64_t seq, float *out);
/* QTensor::add_scaled_row (qtensor.rs:516-543). */
void uto_add_scaled_row(int fmt, const void *payload, const float *scales,
                        int64_t out_dim, int64_t in_dim, int64_t row,
                        float factor, float *acc);
/* QTensor::matvec_rows (qtensor.rs:548-586). */
void uto_matvec_rows(int fmt, const void *payload, const float *scales,
                     int64_t out_dim, int64_t in_dim, int64_t row0,
                     int64_t nrows, const float *x, float *out);

/* --------------------------------------------------------------- math ---- */
/* rmsnorm / softmax / sigmoid / silu (undertow-quant/src/lib.rs:91-123). */
void  uto_rmsnorm(float *out, const float *x, const float *w, int64_t n, float eps);
void  uto_softmax(float *x, int64_t n);
float uto_sigmoid(float x);
float uto_silu(float x);
/* rope_interleave (adapters/undertow-deepseek-moe/src/attention.rs:106-118). */
void  uto_rope_interleave(float *v, int64_t pos, int64_t dim, float theta);
/* argmax (undertow-core/src/sample.rs:353-361). */
int64_t uto_argmax(const float *v, int64_t n);
/* topk_indices (undertow-core/src/router.rs:136-163); returns count. */
int64_t uto_topk_indices(const float *v, int64_t n, int64_t k, int64_t *out);
/* DeepseekSigmoidRouter::route (adapters/.../router.rs:58-113).
 * bias may be NULL.  Writes k expert ids and weights in choice order. */
void uto_route(const float *logits, const float *bias, int64_t n_experts,
               int64_t top_k, int64_t n_group, int64_t topk_group,
               int norm_topk_prob, float routed_scaling_factor,
               int64_t *ids, float *weights);

/* ------------------------------------------------------ expert FFN ------- */
/* One routed expert block over M rows, the body of moe_forward
 * (adapters/.../model.rs:210-281) without the router and shared expert:
 * out[s] = sum_c w[s,c] * down(silu(gate x_s) * up x_s) in choice order.
 * Expert e's gate/up/down payloads live at base + e*stride.  out is zeroed
 * first (the caller's zeroed moe_out, model.rs:167,511). */
void uto_moe_experts(int fmt, int64_t hidden, int64_t inter,
                     const uint8_t *gate_payload, const float *gate_scales,
                     const uint8_t *up_payload, const float *up_scales,
                     const uint8_t *down_payload, const float *down_scales,
                     int64_t M, int64_t top_k, const int64_t *ids,
                     const float *weights, const float *x, float *out);
/* MlpWeights::forward_add (model.rs:43-58): out += down(silu(g)*u). */
void uto_mlp_forward_add(int fmt, int64_t hidden, int64_t inter,
                         const void *gate_payload, const float *gate_scales,
                         const void *up_payload, const float *up_scales,
                         const void *down_payload, const float *down_scales,
                         const float *x, int64_t seq, float *out);

/* ------------------------------------------------------------ MLA core --- */
/* The absorbed score/softmax/context loops of mla_forward_cached
 * (attention.rs:214-234), for precomputed qabs/q_rope:
 *   for row s, head h: n_ctx = pos_base + s + 1,
 *   score_t = (qabs.lat_t + q_rope.krot_t) * scale, softmax, clat = sum p lat.
 * qabs [R,H,L], q_rope [R,H,P], latent [T,L], krot [T,P], clat [R,H,L]. */
void uto_mla_attend(const float *qabs, const float *q_rope, const float *latent,
                    const float *krot, int64_t R, int64_t H, int64_t L,
                    int64_t P, int64_t pos_base, float scale, float *clat);

/* ------------------------------------------------ checkpoint + model ----- */
/* OracleSpec (undertow-bench/src/oracle.rs:17-75) plus the DeepseekConfig
 * fields the forward pass reads (config.rs:30-85).  q_lora_rank == 0 means
 * the Direct q_proj path. */
typedef struct {
    uint64_t seed;
    int64_t vocab_size, hidden_size, intermediate_size, moe_intermediate_size;
    int64_t num_hidden_layers, first_k_dense_replace, num_attention_heads;
    int64_t n_routed_experts, num_experts_per_tok, n_shared_experts;
    int64_t n_group, topk_group;
    int32_t norm_topk_prob;
    float routed_scaling_factor;
    int64_t q_lora_rank, kv_lora_rank, qk_nope_head_dim, qk_rope_head_dim, v_head_dim;
    float rms_norm_eps, rope_theta, init_std;
    int32_t mtp;
    int64_t max_position_embeddings;
} uto_spec;

void uto_spec_default(uto_spec *s);

typedef struct uto_ckpt uto_ckpt;
/* generate_oracle (oracle.rs:150-310): tensors in generation order. */
uto_ckpt *uto_generate(const uto_spec *s);
void      uto_ckpt_free(uto_ckpt *c);
/* write_safetensors (undertow-io/src/writer.rs:73-110,233-239) into buf.
 * Returns the byte count; pass buf=NULL to query the size. */
int64_t   uto_ckpt_safetensors(const uto_ckpt *c, uint8_t *buf, int64_t cap);
/* Per-row quantization of every 2-D tensor by classify_tensor
 * (adapters/.../naming.rs:28-73; convert/src/lib.rs:133-158,229-248). */
int       uto_ckpt_convert(uto_ckpt *c, int expert_fmt, int dense_fmt);
int64_t   uto_ckpt_count(const uto_ckpt *c);
/* Tensor i: name, format, shape; returns 0 or -1. */
int       uto_ckpt_info(const uto_ckpt *c, int64_t i, char *name, int64_t name_cap,
                        int32_t *fmt, int64_t *shape /*[2]*/, int32_t *ndim);
/* Payload bytes (f32 data, int8 codes, packed int4) and scales pointers. */
const void  *uto_ckpt_payload(const uto_ckpt *c, int64_t i, int64_t *nbytes);
const float *uto_ckpt_scales(const uto_ckpt *c, int64_t i);
/* An empty checkpoint, and a copy of one tensor added to it (1-D f32 or
 * 2-D [d0, d1] in fmt; nbytes must equal payload_bytes, scales [d0] for the
 * integer formats).  Returns 0 or -1.  For hand-built test models. */
uto_ckpt *uto_ckpt_new(void);
int       uto_ckpt_add(uto_ckpt *c, const char *name, int32_t fmt, int32_t ndim, int64_t d0,
                       int64_t d1, const void *payload, int64_t nbytes, const float *scales);
/* Test inputs at DeepSeek-V3 width: uto_generate's tensor list with every
 * matrix filled from a counter-based generator (fast, parallel) in the
 * format classify_tensor gives it: codes uniform over the format's range,
 * per-row scales |N(0,std)|/qmax, f32 matrices N(0,std).  Not the
 * reference's generator; a source of seeded weights only. */
uto_ckpt *uto_ckpt_synthesize(const uto_spec *s, uint64_t seed, float std, int expert_fmt,
                              int dense_fmt);

typedef struct uto_model uto_model;
typedef struct uto_session uto_session;
/* load_model_with + ResidentStore (adapters/.../loader.rs:181-302). */
uto_model *uto_model_new(const uto_ckpt *c, const uto_spec *s);
void       uto_model_free(uto_model *m);
/* InferenceSession (model.rs:407-564).  path: 0 Auto, 1 Absorbed,
 * 2 Reconstruct (attention.rs:97-103). */
uto_session *uto_session_new(uto_model *m, int path);
void         uto_session_free(uto_session *s);
/* prefill: returns 0, -1 empty, -2 context overflow, -3 bad token. */
int     uto_session_prefill(uto_session *s, const int32_t *ids, int64_t n, float *logits);
void    uto_session_truncate(uto_session *s, int64_t len);
int64_t uto_session_position(const uto_session *s);
/* on_token (core/model.rs:139-166, mtp.rs:194-314): return 0 to stop. */
typedef int32_t (*uto_token_fn)(void *user, int32_t token);
/* draft_fn of speculative_loop (mtp.rs:263-314): consumed tokens [n], the
 * emitted not-yet-consumed `next`; writes `depth` drafts; < 0 aborts. */
typedef int32_t (*uto_draft_fn)(void *user, const int32_t *tokens, int64_t n, int32_t next,
                                int32_t depth, int32_t *drafts);
/* undertow_core::generate with a greedy sampler (core/model.rs:139-166):
 * stops after a token in stops[] (emitted and counted), when on_token
 * (may be NULL) returns 0, at max_new, or at the context end.  Returns the
 * count or a negative error. */
int64_t uto_generate_greedy(uto_model *m, const int32_t *prompt, int64_t n, int64_t max_new,
                            const int32_t *stops, int64_t n_stops, uto_token_fn on_token,
                            void *user, int32_t *out);
/* greedy_decode (core/model.rs:168-185) without stop ids. */
int64_t uto_greedy_decode(uto_model *m, const int32_t *prompt, int64_t n,
                          int64_t max_new, int32_t *out);
/* MtpState (mtp.rs:48-55) and draft_logits (mtp.rs:74-133): feeds the
 * session's pending positions to the MTP layer and writes the head's
 * logits [vocab] for the last; last_out (may be NULL) gets that position's
 * MTP-layer output row (before the head's norm).  Returns 0, -4 without an
 * MTP head, -5 with nothing pending. */
typedef struct uto_mtp_state uto_mtp_state;
uto_mtp_state *uto_mtp_state_new(void);
void           uto_mtp_state_free(uto_mtp_state *st);
int            uto_draft_logits(uto_model *m, uto_session *s, uto_mtp_state *st,
                                int32_t next_token, float *logits, float *last_out);
/* speculative_loop (mtp.rs:263-314) at depth 1 (the reference) to 3 (an
 * extension: native drafts chain the MTP layer on its own last output row,
 * depth+1 verify rows, longest matching prefix accepted, rollback to the
 * last verified position).  draft_fn NULL: the native MTP head.  Stop and
 * callback rules of uto_generate_greedy.  Returns the produced count. */
int64_t uto_speculative_loop(uto_model *m, const int32_t *prompt, int64_t n, int64_t max_new,
                             int32_t depth, const int32_t *stops, int64_t n_stops,
                             uto_token_fn on_token, void *user, uto_draft_fn draft_fn,
                             void *draft_user, int32_t *out, int64_t *drafted, int64_t *accepted);
/* generate_greedy_mtp (mtp.rs:176-191) without stop ids: depth 1. */
int64_t uto_generate_mtp(uto_model *m, const int32_t *prompt, int64_t n,
                         int64_t max_new, int32_t *out, int64_t *drafted,
                         int64_t *accepted);

#ifdef __cplusplus
}
#endif
#endif
