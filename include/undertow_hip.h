/*
 * undertow_hip.h -- C ABI of the MI355X (gfx950) backend for undertow's
 * MTP draft+verify decode step.
 *
 * Every entry point is plain C: integer status codes, plain pointers and
 * sizes.  Pointers named *_dev are device (HBM) addresses; every other
 * pointer is host memory that is only read (or written) during the call.
 * Work is enqueued on the context's HIP stream; entry points that return
 * host-visible results synchronise that stream before returning.
 *
 * Each declaration names the reference routine (mohitmishra786/undertow,
 * Rust) whose semantics it reproduces and whose call site a Rust binding in
 * undertow-quant / adapters/undertow-deepseek-moe would route through it.
 *
 * Threading: a ut_ctx (one HIP stream) belongs to one thread at a time and
 * is not internally synchronised.  ut_qtensor / ut_expert_table / ut_model
 * handles are immutable after set-up and may be shared by contexts on the
 * same device.  Sessions are per thread, like the reference's
 * InferenceSession (adapters/undertow-deepseek-moe/src/model.rs:407-445).
 */
#ifndef UNDERTOW_HIP_H
#define UNDERTOW_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- status */
/* Replaces the reference's panics (assert_eq! in QTensor::matmul,
 * undertow-quant/src/qtensor.rs:283-284) and EngineError variants
 * (undertow-core/src/error.rs:6-37).  No exception or abort crosses the ABI;
 * ut_last_error() gives the message of the last failure on a context. */
enum {
    UT_OK = 0,
    UT_ERR_ARG = -1,              /* null handle / pointer, bad enum value */
    UT_ERR_SHAPE = -2,            /* x / out length does not match the tensor */
    UT_ERR_FORMAT = -3,           /* payload size matches neither int8 nor int4 */
    UT_ERR_OOM = -4,              /* device or host allocation failed */
    UT_ERR_HIP = -5,              /* a HIP runtime call failed */
    UT_ERR_BAD_EXPERT = -6,       /* expert id out of range or not loaded */
    UT_ERR_CONTEXT_OVERFLOW = -7, /* EngineError::ContextOverflow */
    UT_ERR_BAD_TOKEN = -8,        /* token id >= vocab_size */
    UT_ERR_NOT_FOUND = -9,        /* a required tensor was never set */
    UT_ERR_STATE = -10,           /* call out of order (e.g. no MTP head) */
    UT_ERR_IO = -11               /* EngineError::Io: a checkpoint file could not be read */
};

/* QuantFormat (undertow-quant/src/qtensor.rs:17-21).  UT_FMT_INFER asks
 * ut_qtensor_upload to deduce int8/int4 from the payload size, as
 * read_qtensor does (undertow-io/src/reader.rs:421-430). */
enum { UT_FMT_INFER = -1, UT_FMT_F32 = 0, UT_FMT_INT8 = 1, UT_FMT_INT4 = 2 };

typedef struct ut_ctx ut_ctx;
typedef struct ut_qtensor ut_qtensor;
typedef struct ut_expert_table ut_expert_table;
typedef struct ut_model ut_model;
typedef struct ut_session ut_session;

/* --------------------------------------------------------------- context */
/* No reference counterpart (the reference has no device): owns one HIP
 * stream on `device` and a scratch arena reused across calls. */
int32_t     ut_ctx_create(int32_t device, ut_ctx **out);
void        ut_ctx_destroy(ut_ctx *ctx);
const char *ut_last_error(const ut_ctx *ctx);
/* Run subsequent work on `stream`, a hipStream_t of the same device (e.g.
 * torch.cuda.current_stream().cuda_stream); NULL is the null stream.  The
 * context's own stream is what ut_ctx_stream() returns right after
 * ut_ctx_create().  Handles may be released in any order: a session keeps
 * its model alive and a model its context until they are released. */
int32_t     ut_ctx_set_stream(ut_ctx *ctx, void *stream);
void       *ut_ctx_stream(ut_ctx *ctx);
/* Waits for the context's stream; also reports errors detected on device
 * since the last call (UT_ERR_BAD_EXPERT). */
int32_t     ut_ctx_synchronize(ut_ctx *ctx);
/* Per-kernel timing with HIP events on the context stream (bench tooling):
 * while enabled, every kernel the library launches is bracketed by events;
 * ut_ctx_kernel_time() reports launches and total milliseconds of the
 * kernels whose name starts with `prefix`. */
int32_t     ut_ctx_enable_timing(ut_ctx *ctx, int32_t on);
int32_t     ut_ctx_kernel_time(ut_ctx *ctx, const char *prefix, int64_t *launches,
                               double *total_ms);

/* Measurement helper (no counterpart in the reference; for roofline
 * calibration): streams `bytes` of device memory at buf_dev with
 * non-temporal 16-byte loads, `reps` times on the context's stream, and
 * returns the read rate in GB/s.  bytes must be a positive multiple of 16
 * and buf_dev 16-byte aligned. */
int32_t     ut_probe_read_bandwidth(ut_ctx *ctx, const void *buf_dev, int64_t bytes, int32_t reps,
                                    double *gbs);
/* The same read kernel over `reps` consecutive windows of window_bytes in
 * turn (wrapping within total_bytes >= 2 windows), one launch each, so that
 * with total_bytes well above the 256 MB memory-side cache every launch
 * reads data fresh from HBM: the single-launch read floor for a kernel of
 * that size.  window_bytes a multiple of 256. */
int32_t     ut_probe_read_windows(ut_ctx *ctx, const void *buf_dev, int64_t total_bytes,
                                  int64_t window_bytes, int32_t reps, double *gbs);

/* --------------------------------------------------------------- QTensor */
/* QTensor::from_quantized (undertow-quant/src/qtensor.rs:85-138) /
 * read_qtensor (undertow-io/src/reader.rs:403-444): copies the payload
 * (host or device memory)
 * (f32 data, int8 codes, or int4 rows of ceil(in/2) bytes, low nibble =
 * even index) and per-output-row scales to HBM.  Validates payload_len
 * against QuantFormat::payload_bytes (qtensor.rs:43-49) and
 * scales_len == out_dim (int formats; ignored for f32). */
int32_t ut_qtensor_upload(ut_ctx *ctx, int32_t fmt, const void *payload, int64_t payload_len,
                          const float *scales, int64_t scales_len, int64_t out_dim,
                          int64_t in_dim, ut_qtensor **out);
void    ut_qtensor_free(ut_qtensor *qt);
/* QTensor::format / out_dim / in_dim / nbytes (qtensor.rs:215-248). */
int32_t ut_qtensor_format(const ut_qtensor *qt);
int64_t ut_qtensor_out_dim(const ut_qtensor *qt);
int64_t ut_qtensor_in_dim(const ut_qtensor *qt);
int64_t ut_qtensor_nbytes(const ut_qtensor *qt);
/* QTensor::quantize (undertow-quant/src/qtensor.rs:142-213) on the device:
 * the f32 matrix w_dev [out_dim, in_dim] becomes a new QTensor of format
 * fmt with per-row s = max|w|/qmax (qmax 127 / 7) and codes
 * round(w/s) (half away from zero) clamped to +-qmax; a row of zeros keeps
 * s = 0.  Bit-exact with the reference.  A non-finite weight is the
 * reference's Err: UT_ERR_FORMAT, the message naming its flat index, row
 * and column (the smallest such index). */
int32_t ut_qtensor_quantize(ut_ctx *ctx, int32_t fmt, const float *w_dev, int64_t out_dim,
                            int64_t in_dim, ut_qtensor **out);
/* The QTensor's stored data read back to the host, as TensorEntry::
 * from_qtensor reads a QTensor's payload and scales to write them
 * (undertow-io/src/writer.rs:35-64): payload_host gets payload_len bytes
 * (must equal QuantFormat::payload_bytes), scales_host out_dim floats
 * (NULL for f32 tensors).  Synchronises the context's stream. */
int32_t ut_qtensor_download(ut_ctx *ctx, const ut_qtensor *qt, void *payload_host,
                            int64_t payload_len, float *scales_host);
/* QTensor::dequantize (qtensor.rs:265-272): out[o,i] = fl(scale[o]*q[o,i])
 * (bit-exact), f32 tensors copied.  out_dev holds out_dim*in_dim floats. */
int32_t ut_qtensor_dequantize(ut_ctx *ctx, const ut_qtensor *qt, float *out_dev);
/* QTensor::matmul(&self, out, x, seq) (qtensor.rs:281-319):
 * out[s,o] = scale[o] * sum_i x[s,i]*q[o,i], x [seq,in] and out [seq,out]
 * row-major f32.  x_len / out_len are element counts, checked like the
 * reference's assert_eq!s.  Each output row's value does not depend on seq
 * (the reference's "threading never changes numerics"). */
int32_t ut_qtensor_matmul(ut_ctx *ctx, const ut_qtensor *qt, float *out_dev, int64_t out_len,
                          const float *x_dev, int64_t x_len, int64_t seq);
/* set_fast_int8 / fast_int8_enabled (undertow-quant/src/lib.rs:31-43): the
 * opt-in fast path for int8 matmuls, per context here (the reference's
 * switch is process-global).  While on, ut_qtensor_matmul and
 * ut_qtensor_matvec_rows on int8 tensors quantise each activation row to i8
 * with one scale (quantize_activations, lib.rs:46-59) and take the exact
 * integer dot (avx512.rs:221-242, neon.rs:139-184):
 * out = (acc as f32) * a_scale * scale[o].  It changes numerics (about 1e-2
 * relative; the reference bounds it at 3% of the row magnitude) and is off
 * by default.  The model's own projections and the expert block keep exact
 * numerics. */
int32_t ut_set_fast_int8(ut_ctx *ctx, int32_t enabled);
int32_t ut_fast_int8_enabled(const ut_ctx *ctx);
/* QTensor::add_scaled_row (qtensor.rs:516-543): acc[i] += (factor*scale[row])*q[row,i]. */
int32_t ut_qtensor_add_scaled_row(ut_ctx *ctx, const ut_qtensor *qt, int64_t row, float factor,
                                  float *acc_dev);
/* QTensor::matvec_rows (qtensor.rs:548-586): out[j] = scale[row0+j] *
 * sum_i x[i]*q[row0+j, i] for j in [0, nrows), x [in_dim] and out [nrows]
 * f32 on the device.  x_len / out_len are element counts, checked like the
 * reference's assert!s (UT_ERR_SHAPE, also when row0 + nrows > out_dim). */
int32_t ut_qtensor_matvec_rows(ut_ctx *ctx, const ut_qtensor *qt, int64_t row0, int64_t nrows,
                               const float *x_dev, int64_t x_len, float *out_dev,
                               int64_t out_len);

/* ---------------------------------------------------------------- router */
/* RouterAdapter::route (undertow-core/src/adapter.rs:99-114) as
 * DeepseekSigmoidRouter::route (adapters/undertow-deepseek-moe/src/
 * router.rs:58-113) over `rows` rows of gate logits [rows, n_experts]:
 * sigmoid, + correction bias (bias_dev may be NULL) for selection only,
 * group limitation by the sum of each group's top-2, top-k by
 * topk_indices (undertow-core/src/router.rs:136-163, lowest index first on
 * ties), weights = sigmoid normalised (norm_topk_prob) and scaled.
 * Writes ids [rows, top_k] int32 and weights [rows, top_k] in choice order. */
int32_t ut_route(ut_ctx *ctx, const float *logits_dev, const float *bias_dev, int64_t rows,
                 int64_t n_experts, int32_t top_k, int32_t n_group, int32_t topk_group,
                 int32_t norm_topk_prob, float routed_scaling_factor, int32_t *ids_dev,
                 float *weights_dev);

/* ----------------------------------------------------------- expert block */
/* Device-side counterpart of the expert store (TieredStore::get_expert,
 * undertow-core/src/store.rs:142-162; ResidentStore :167-229): per expert
 * the gate/up [inter, hidden] and down [hidden, inter] QTensors.  The table
 * borrows the QTensor handles; they must outlive it. */
int32_t ut_expert_table_create(ut_ctx *ctx, int64_t n_experts, int64_t hidden, int64_t inter,
                               ut_expert_table **out);
int32_t ut_expert_table_set(ut_expert_table *tbl, int64_t expert, const ut_qtensor *gate,
                            const ut_qtensor *up, const ut_qtensor *down);
void    ut_expert_table_free(ut_expert_table *tbl);
/* The routed-expert body of moe_forward (adapters/undertow-deepseek-moe/
 * src/model.rs:210-281) for `rows` rows already routed on device:
 * out[s] = sum_c weights[s,c] * down(silu(gate x_s) * up x_s) over the
 * choices c in router order (out is overwritten, i.e. starts at zero).
 * Each unique expert's weights are read once for all rows that chose it.
 * Experts must all share one format (int4 or int8).  Expert ids are
 * validated on device without a host round trip: an id out of range or not
 * loaded contributes nothing, and UT_ERR_BAD_EXPERT is returned by the next
 * ut_ctx_synchronize() on this context. */
int32_t ut_moe_experts(ut_ctx *ctx, const ut_expert_table *tbl, const int32_t *ids_dev,
                       const float *weights_dev, int64_t rows, int32_t top_k, const float *x_dev,
                       float *out_dev);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops and harnesses that
 * forbid hipMalloc): ut_moe_experts with the same arguments and results,
 * allocating nothing.  Its working memory (slot plan, h, digits, down
 * outputs) is a fixed 32 MiB array per device in the library's code
 * object, looked up when the context is created; calls whose working set
 * exceeds it (about top_k * 4 rows * (hidden + inter) * 4 bytes, e.g.
 * top_k 64 at hidden 7168) return UT_ERR_ARG.  Every call on one GPU shares
 * that array: the first context to call owns it until it is destroyed, and
 * calls from any other context on that GPU return UT_ERR_STATE.  The
 * owner's calls are ordered on its stream; a caller that runs them on
 * several streams itself (ut_ctx_set_stream between overlapping calls
 * synchronises) must not let two overlap. */
int32_t ut_moe_experts_noalloc(ut_ctx *ctx, const ut_expert_table *tbl, const int32_t *ids_dev,
                               const float *weights_dev, int64_t rows, int32_t top_k,
                               const float *x_dev, float *out_dev);

/* Route then run the routed experts, as moe_forward does per row
 * (adapters/undertow-deepseek-moe/src/model.rs:210-281: route at :210-216,
 * then the expert body): the choices of ut_route over logits_dev [rows, E]
 * (E = the table's expert count; same arguments and semantics) are written
 * to ids_dev / weights_dev [rows, top_k], and out_dev is ut_moe_experts'
 * result for them.  Results are identical to ut_route followed by
 * ut_moe_experts; at one row with the one-wave router's shapes the routing
 * runs inside the expert launch. */
int32_t ut_moe_route_experts(ut_ctx *ctx, const ut_expert_table *tbl, const float *logits_dev,
                             const float *bias_dev, int64_t rows, int32_t top_k, int32_t n_group,
                             int32_t topk_group, int32_t norm_topk_prob,
                             float routed_scaling_factor, const float *x_dev, float *out_dev,
                             int32_t *ids_dev, float *weights_dev);

/* bf16 activations: ut_moe_experts / ut_moe_route_experts with x_dev as
 * bf16 bits [rows, hidden] (16-byte aligned, hidden % 8 == 0, else
 * UT_ERR_ARG).  Each value is widened to f32 exactly, as the reference
 * loads bf16 tensors (undertow-io/src/reader.rs:261-267 via
 * half::bf16::to_f32), so out is bit-identical to the f32 entry point on
 * the widened x.  At one row the gate/up launch reads the bf16 values
 * itself (half the activation bytes); other shapes widen them in the
 * working memory first. */
int32_t ut_moe_experts_bf16(ut_ctx *ctx, const ut_expert_table *tbl, const int32_t *ids_dev,
                            const float *weights_dev, int64_t rows, int32_t top_k,
                            const uint16_t *x_dev, float *out_dev);
int32_t ut_moe_route_experts_bf16(ut_ctx *ctx, const ut_expert_table *tbl,
                                  const float *logits_dev, const float *bias_dev, int64_t rows,
                                  int32_t top_k, int32_t n_group, int32_t topk_group,
                                  int32_t norm_topk_prob, float routed_scaling_factor,
                                  const uint16_t *x_dev, float *out_dev, int32_t *ids_dev,
                                  float *weights_dev);

/* ------------------------------------------------------ sample / verify */
/* argmax (undertow-core/src/sample.rs:353-361) per row: first index of the
 * maximum; NaN never wins; returns 0 when row[0] is NaN. */
int32_t ut_argmax_rows(ut_ctx *ctx, const float *logits_dev, int64_t rows, int64_t vocab,
                       int32_t *idx_dev);

/* ------------------------------------------------------------ attention */
/* The absorbed score/softmax/context loops of mla_forward_cached
 * (adapters/undertow-deepseek-moe/src/attention.rs:214-234) for R query
 * rows x H heads: row s sees n_ctx = pos_base + s + 1 cache positions,
 * score_t = (qabs.latent_t + q_rope.krot_t) * scale, fp32 softmax,
 * clat = sum_t p_t latent_t.  qabs [R,H,L], q_rope [R,H,P], latent [T,L],
 * krot [T,P] (T >= pos_base + R), clat [R,H,L]; all f32. */
int32_t ut_mla_attend(ut_ctx *ctx, const float *qabs_dev, const float *q_rope_dev,
                      const float *latent_dev, const float *krot_dev, int64_t R, int64_t H,
                      int64_t L, int64_t P, int64_t pos_base, float scale, float *clat_dev);

/* The same attention over a cache kept on the device in the split form the
 * bf16 matrix-core kernel reads (LayerKvCache, attention.rs:76-94, held as
 * [T][2][L+P] bf16: per position the hi parts of [latent | krot], then the lo
 * parts, x = hi + lo to about 2^-17 |x|; the bytes of the f32 cache).
 * ut_mla_cache_split converts T f32 positions into that form (kc_dev holds
 * T * 2 * (L+P) bf16, 16-byte aligned); ut_mla_attend_split then attends
 * without converting.  Shapes: H % 32 == 0, L == 512, P == 64 (DeepSeek-V3);
 * others return UT_ERR_SHAPE. */
int32_t ut_mla_cache_split(ut_ctx *ctx, const float *latent_dev, const float *krot_dev, int64_t T,
                           int64_t L, int64_t P, void *kc_dev);
int32_t ut_mla_attend_split(ut_ctx *ctx, const float *qabs_dev, const float *q_rope_dev,
                            const void *kc_dev, int64_t R, int64_t H, int64_t L, int64_t P,
                            int64_t pos_base, float scale, float *clat_dev);

/* ---------------------------------------------------------------- model */
/* DeepseekConfig fields the forward pass reads (adapters/undertow-deepseek-
 * moe/src/config.rs:30-85).  q_lora_rank == 0 selects the direct q_proj. */
typedef struct {
    int64_t vocab_size, hidden_size, intermediate_size, moe_intermediate_size;
    int64_t num_hidden_layers, first_k_dense_replace, num_attention_heads;
    int64_t n_routed_experts, num_experts_per_tok, n_shared_experts;
    int64_t n_group, topk_group;
    int32_t norm_topk_prob;
    float routed_scaling_factor;
    int64_t q_lora_rank, kv_lora_rank, qk_nope_head_dim, qk_rope_head_dim, v_head_dim;
    float rms_norm_eps, rope_theta;
    int32_t mtp;                      /* 1: load the MTP module at layer index num_hidden_layers */
    int64_t max_position_embeddings;  /* context capacity of a session */
} ut_model_config;

/* load_model_with (adapters/undertow-deepseek-moe/src/loader.rs:181-302),
 * split into create / set_tensor / finalize so a host loader streams
 * tensors straight from its shards.  Tensor names are the checkpoint's
 * (model.layers.N.self_attn.q_a_proj.weight, ...).  set_tensor takes a 2-D
 * matrix [d0, d1] in any format (fmt UT_FMT_INFER: int8/int4 from the
 * payload size, as read_qtensor) or a 1-D f32 vector (d1 == 1 and
 * scales == NULL).  finalize checks that every tensor the config needs is
 * present with the right shape (UT_ERR_NOT_FOUND / UT_ERR_SHAPE). */
int32_t ut_model_create(ut_ctx *ctx, const ut_model_config *cfg, ut_model **out);
int32_t ut_model_set_tensor(ut_model *m, const char *name, int32_t fmt, const void *payload,
                            int64_t nbytes, const float *scales, int64_t d0, int64_t d1);
int32_t ut_model_finalize(ut_model *m);
/* load_model_with's tensor reads (adapters/undertow-deepseek-moe/src/
 * loader.rs:67-229 through read_qtensor and ShardedModelReader, undertow-io/
 * src/reader.rs:78-143,300-444) straight into HBM, then finalize: opens
 * dir/model.safetensors.index.json (or a single dir/model.safetensors),
 * validates every shard header (known dtype, data_offsets consistent with
 * shape and dtype, extents inside the file, header <= 100 MB), and streams
 * each tensor the config needs into one device arena: pread into pinned
 * staging buffers, two in flight, each drained by hipMemcpyAsync.
 * Quantized weights are the converter's `<name>` U8 payload plus
 * `<name>.scales` F32 [out_dim] (int8 or int4 from the payload size, as
 * read_qtensor); plain tensors may be F32, BF16 or F16 (widened to f32).
 * Errors: UT_ERR_IO (unreadable file), UT_ERR_FORMAT (bad header or
 * payload size), UT_ERR_NOT_FOUND, UT_ERR_SHAPE.  bytes_read (may be NULL)
 * gets the tensor bytes read from disk.  Needs a fresh model. */
int32_t ut_model_load_dir(ut_model *m, const char *dir, int64_t *bytes_read);
/* The HBM tier of the expert store: DiskExpertStore with an LRU or weighted
 * ExpertCache (undertow-io/src/store.rs:46-249, undertow-core/src/cache.rs:
 * 15-340) whose cache lives in device memory.  Routed experts stay in the
 * backing source; a byte-budgeted pool of HBM slots holds the cached ones
 * (one slot = one expert's gate, up and down payloads and scales), plus
 * room for the experts of one step beyond the budget.  Each MoE step routes
 * on the device, reads the choices back, loads missing experts into slots
 * (evicting by the policy; pinned experts stay) and publishes the layer's
 * pointer table before the expert launches: results are bit-identical to a
 * resident model.  prefetch: at one-row decode, a pilot routing of the next
 * MoE layer on the post-attention residual (pilot_prefetch, adapters/
 * undertow-deepseek-moe/src/model.rs:290-318) loads its predicted experts
 * during the current step. */
typedef struct {
    int64_t hbm_budget_bytes; /* cache_budget_bytes for routed experts */
    int32_t policy;           /* CachePolicy: 0 LRU, 1 weighted (half-life 512 accesses) */
    int32_t prefetch;         /* 1: pilot-router prefetch one layer ahead at decode */
} ut_expert_store_config;
/* StoreStatsSnapshot (undertow-core/src/store.rs). */
typedef struct {
    int64_t hits, misses, bytes_read, evictions, prefetch_issued, prefetch_dropped;
    int64_t bytes_used, budget_bytes, pinned_experts;
    double read_seconds;
} ut_store_stats;
/* load_model_with with StoreChoice::DiskStreaming (adapters/undertow-
 * deepseek-moe/src/loader.rs:233-302): ut_model_load_dir for everything but
 * the routed experts, which stay in dir's shards behind the HBM tier
 * (pread into pinned staging on a miss, read_qtensor's layout). */
int32_t ut_model_load_dir_tiered(ut_model *m, const char *dir, const ut_expert_store_config *cfg,
                                 int64_t *bytes_read);
/* Benchmark support, no reference counterpart: ut_model_synthesize with the
 * routed experts behind the HBM tier, served from a pinned host pool of
 * host_pool_experts seeded experts (key (layer, e) reads pool entry
 * (layer * E + e) mod host_pool_experts). */
int32_t ut_model_synthesize_tiered(ut_model *m, uint64_t seed, float init_std, int32_t expert_fmt,
                                   int32_t dense_fmt, const ut_expert_store_config *cfg,
                                   int64_t host_pool_experts);
/* DiskExpertStore::pin_hottest (store.rs:146-166): loads and pins the
 * (layer, expert) pairs in order (hottest first, as ExpertProfile::hottest)
 * until budget_bytes are pinned or the cache's budget is full of pins;
 * out-of-range pairs are skipped. */
int32_t ut_model_pin_experts(ut_model *m, const int32_t *layer_expert, int64_t n,
                             int64_t budget_bytes, int64_t *pinned_bytes);
/* TieredStore::stats (store.rs:233-240).  UT_ERR_STATE without a store. */
int32_t ut_model_store_stats(ut_model *m, ut_store_stats *out);
/* TieredStore::usage (store.rs:222-231): per-expert get counts
 * [num_hidden_layers (+1 with MTP)][n_routed_experts], the data of an
 * ExpertProfile (undertow-core/src/profile.rs:18-100). */
int32_t ut_model_expert_usage(ut_model *m, int64_t *counts, int64_t n);
/* Benchmark support, no reference counterpart: fills every tensor of the
 * config on device from a counter-based generator (int4 experts and int8
 * dense matrices with codes uniform over the format's range and per-row
 * scales |N(0,std)|/qmax; norms 1 +- 0.1; router gate f32 N(0,std); bias
 * ramp -0.1..0.1) and finalizes.  expert_fmt / dense_fmt: UT_FMT_INT4 or
 * UT_FMT_INT8. */
int32_t ut_model_synthesize(ut_model *m, uint64_t seed, float init_std, int32_t expert_fmt,
                            int32_t dense_fmt);
/* Benchmark support, no reference counterpart: ut_model_synthesize with
 * construction flags.  UT_SYNTH_MTP_RESTATES builds a model whose MTP head
 * predicts like the main model, as a trained head does (random weights
 * otherwise accept almost no drafts): the MTP module's layer restates the
 * first MoE layer (the same bytes) and its head and head norm the lm_head
 * and final norm; the other layers' residual writes (o_proj and the down
 * projections) get scales 2^-10 of the synthesized ones; embedding rows
 * get unit RMS and eh_proj = [I | 0], so the MTP module sees the next
 * token's embedding as the main model does.  The weight bytes and shapes
 * are the config's.  Needs an MTP module, int8 dense weights and at least
 * one MoE layer (else UT_ERR_ARG). */
enum { UT_SYNTH_MTP_RESTATES = 1 };
int32_t ut_model_synthesize_ex(ut_model *m, uint64_t seed, float init_std, int32_t expert_fmt,
                               int32_t dense_fmt, int32_t flags);
int64_t ut_model_device_bytes(const ut_model *m);
/* LoadOptions::kv_budget_bytes (undertow-core/src/model.rs:36-61) and the
 * effective context it gives (adapters/undertow-deepseek-moe/src/
 * loader.rs:311-325, Model::max_context at model.rs:362-364): per position
 * num_hidden_layers * (kv_lora_rank + qk_rope_head_dim) * 4 bytes plus,
 * with an MTP head, hidden_size * 4 + 8; the context is
 * min(max_position_embeddings, max(budget / that, 1)).  Sessions created
 * afterwards hold that many positions and report UT_ERR_CONTEXT_OVERFLOW
 * beyond it.  A negative budget removes the bound; 0 is UT_ERR_ARG. */
int32_t ut_model_set_kv_budget(ut_model *m, int64_t kv_budget_bytes);
int64_t ut_model_max_context(const ut_model *m);
void    ut_model_free(ut_model *m);

/* InferenceSession (model.rs:407-564).  path: 0 = Auto, 1 = Absorbed,
 * 2 = Reconstruct (attention.rs:97-103); this backend runs the absorbed
 * form for every path (the reference's two paths agree to < 1e-4,
 * attention.rs:362-422). */
int32_t ut_session_create(ut_model *m, int32_t path, ut_session **out);
/* A session whose work runs on `ctx` (its stream, scratch and staging), a
 * context on the model's device other than the model's own, so that
 * sessions on several threads share one model without sharing a stream:
 * the reference's Session per thread over an Arc'd model
 * (undertow-bench/tests/pipeline.rs:226-249).  ctx NULL: the model's.
 * The session holds a reference to ctx until it is freed.  A model whose
 * routed experts sit behind the HBM tier serves sessions on its own
 * context only (UT_ERR_STATE). */
int32_t ut_session_create_on(ut_model *m, ut_ctx *ctx, int32_t path, ut_session **out);
void    ut_session_free(ut_session *s);
/* InferenceSession::prefill (model.rs:447-547): runs ids[0..n) through the
 * model, extends the KV cache.  logits_host [n, vocab] may be NULL;
 * argmax_host [n] (per-row argmax computed on device) may be NULL.
 * Errors: UT_ERR_ARG (n == 0), UT_ERR_CONTEXT_OVERFLOW, UT_ERR_BAD_TOKEN. */
int32_t ut_session_prefill(ut_session *s, const int32_t *ids, int64_t n, float *logits_host,
                           int32_t *argmax_host);
/* InferenceSession::truncate (model.rs:556-564). */
int32_t ut_session_truncate(ut_session *s, int64_t len);
int64_t ut_session_position(const ut_session *s);

/* DeepseekMoeModel::stop_ids (adapters/undertow-deepseek-moe/src/
 * loader.rs:304-309, model.rs:93): the checkpoint's stop tokens (config
 * eos ids plus generation_config's), which every generation call below
 * honours.  Empty until set. */
int32_t ut_model_set_stop_ids(ut_model *m, const int32_t *ids, int64_t n);

/* No reference counterpart (the reference runs on the CPU): the one-row
 * decode steps of the greedy loop (ut_generate) and the verify steps of the
 * MTP loop (ut_generate_mtp / ut_speculative_loop: depth + 1 rows) replayed
 * from graphs captured on the context's stream, instead of about 40-60
 * kernel launches per step from the host.  Every position-dependent kernel
 * of a step reads the session's position from device memory (reset by one
 * small launch after a rollback), attention grids are sized for the
 * session's capacity (workgroups past the context exit at once), and the
 * step advances the position itself.  Outputs are identical to the eager
 * launches.  A session captures on its second step of each shape; if
 * capturing fails (or the graph would hold anything but kernel launches)
 * the session stays eager.  Not used with the expert tier or kernel timing
 * on.  Off by default. */
int32_t ut_model_enable_graphs(ut_model *m, int32_t on);
/* Counts since the model was made: graphs captured, steps replayed from
 * them, captures given up (each pointer may be NULL). */
int32_t ut_model_graph_stats(const ut_model *m, int64_t *captures, int64_t *replays,
                             int64_t *failures);

/* on_token of undertow_core::generate (undertow-core/src/model.rs:139-166)
 * and of the speculative loops (mtp.rs:194-257, 263-314): called with each
 * emitted token in order; return 0 to end the stream after it. */
typedef int32_t (*ut_token_fn)(void *user, int32_t token);
/* draft_fn of speculative_loop (mtp.rs:263-314): `tokens` are the
 * session's consumed tokens [n_tokens] (prompt plus verified tokens), `next`
 * the emitted token not consumed yet.  Writes `depth` draft ids (the
 * reference drafts one); returns 0, or a negative status that ends the
 * loop with that status. */
typedef int32_t (*ut_draft_fn)(void *user, const int32_t *tokens, int64_t n_tokens, int32_t next,
                               int32_t depth, int32_t *drafts);

/* undertow_core::generate with a greedy sampler (undertow-core/src/
 * model.rs:139-166; greedy_decode :168-185) on a fresh session: emits up to
 * max_new tokens into out and to on_token (may be NULL), stopping after a
 * stop token (the model's stop ids or extra_stop_ids, emitted and counted)
 * or when on_token returns 0.  Returns the count (short of max_new also when
 * the context is full) or a negative status. */
int64_t ut_generate(ut_model *m, const int32_t *prompt, int64_t n, int64_t max_new,
                    const int32_t *extra_stop_ids, int64_t n_extra, ut_token_fn on_token,
                    void *user, int32_t *out);
/* ut_generate without extra stop ids or callback. */
int64_t ut_generate_greedy(ut_model *m, const int32_t *prompt, int64_t n, int64_t max_new,
                           int32_t *out);
/* speculative_loop (adapters/undertow-deepseek-moe/src/mtp.rs:263-314) and
 * generate_greedy_mtp (:176-191).  Drafts come from draft_fn, or from the
 * native MTP head (draft_logits, mtp.rs:74-133) when draft_fn is NULL.
 * depth 1 is the reference: draft one token, verify [next, draft] as a
 * 2-row prefill, accept iff argmax(row 0) == draft, else roll the draft's
 * KV position back.  depth 2..3 (no reference counterpart) drafts 2-3
 * tokens (the native head chains the MTP module on its own last output
 * row), verifies depth+1 rows and accepts the longest matching prefix; the
 * main KV rolls back to the last verified position and the MTP module is
 * only fed verified positions, so the output always equals ut_generate's.
 * Stop ids, on_token and max_new end the stream as in ut_generate, also in
 * the middle of an accepted run.  Returns the produced count; drafted /
 * accepted count draft tokens (MtpStats). */
int64_t ut_speculative_loop(ut_model *m, const int32_t *prompt, int64_t n, int64_t max_new,
                            int32_t depth, const int32_t *extra_stop_ids, int64_t n_extra,
                            ut_token_fn on_token, void *user, ut_draft_fn draft_fn,
                            void *draft_user, int32_t *out, int64_t *drafted, int64_t *accepted);
/* ut_speculative_loop with the native MTP head, no extra stop ids or callback. */
int64_t ut_generate_mtp(ut_model *m, const int32_t *prompt, int64_t n, int64_t max_new,
                        int32_t depth, int32_t *out, int64_t *drafted, int64_t *accepted);
/* draft_logits (mtp.rs:74-133) on the session's MTP state: feeds the
 * positions not yet fed to the MTP layer (t_next = the following consumed
 * token, next_token for the last) and writes the head's logits [vocab] for
 * the last one (logits_host may be NULL) and their argmax (draft_host may
 * be NULL).  UT_ERR_STATE when the model has no MTP head or nothing is
 * pending. */
int32_t ut_session_draft_logits(ut_session *s, int32_t next_token, float *logits_host,
                                int32_t *draft_host);

#ifdef __cplusplus
}
#endif
#endif /* UNDERTOW_HIP_H */
