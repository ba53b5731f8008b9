/*
 * aarambh_hip.h -- C ABI of libaarambh_hip, the MI355X (gfx950) speculative
 * verify path for aarambh-studio.
 *
 * Plain pointers and sizes only.  One context owns one HIP stream, the device
 * copy of one target model (quantised weights, optional MTP heads) and a KV
 * cache with `max_batch` sequence slots.  A context is not thread-safe; calls
 * on one context run in order on its stream.  Every int-returning function
 * returns an aarh_status; aarh_last_error() gives the message of the last
 * failure.
 *
 * Drop-in boundary: this sits at the model + KV level of the reference
 * (model/src/model.rs forward_with_cache_output / forward_mtp_head and
 * inference/src/kvcache.rs), plus the engine loop and the acceptance math,
 * because candle 0.10.2 has no HIP device to plug a CustomOp into
 * (core/src/device.rs:5-12).
 */
#ifndef AARAMBH_HIP_H
#define AARAMBH_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Mirrors AarambhError (core/src/error.rs:5-33): Config, Shape, Unsupported, Checkpoint,
   Io, plus Device. */
typedef enum {
    AARH_OK = 0,
    AARH_ERR_CONFIG = 1,
    AARH_ERR_SHAPE = 2,
    AARH_ERR_UNSUPPORTED = 3,
    AARH_ERR_DEVICE = 4,
    AARH_ERR_CHECKPOINT = 5,
    AARH_ERR_IO = 6
} aarh_status;

/* Weight storage formats (quant/src/types.rs:68-90 plus the build's layouts). */
enum {
    AARH_W_F32 = 0,       /* reference CPU dtype */
    AARH_W_BF16 = 1,
    AARH_W_INT8_ROW = 2,  /* symmetric per-output-channel INT8, f32 row scales */
    AARH_W_INT4_G128 = 3  /* PackedInt4Tensor semantics, group 128, fp16 scale + zero */
};
enum { AARH_KV_F32 = 0, AARH_KV_F16 = 1, AARH_KV_INT8 = 2 };
enum { AARH_T_NORM = 0, AARH_T_LINEAR = 1, AARH_T_EMBED = 2 };
enum { AARH_FINISH_MAX_TOKENS = 0, AARH_FINISH_EOS = 1, AARH_FINISH_CONTEXT_LIMIT = 2 };
/* Near-tie flags: |p/q - u| < 1e-5, |cdf - u| < 1e-6, top-p cumulative within 1e-6 of top_p. */
enum { AARH_FLAG_RATIO_NEAR = 1u, AARH_FLAG_CDF_NEAR = 2u, AARH_FLAG_TOPP_NEAR = 8u };
enum { AARH_TOP_CANDIDATES = 5 };

typedef struct aarh_ctx aarh_ctx;

/* ModelConfig subset (core/src/config.rs:734-776) + MtpConfig (:275-283) + device sizing. */
typedef struct {
    int32_t vocab_size, hidden_dim, ffn_dim, n_layers, n_heads, n_kv_heads, max_seq_len;
    float rope_theta, norm_eps;
    int32_t num_future_tokens; /* MTP horizon; 0 = no MTP heads */
    int32_t weight_format;     /* AARH_W_* for every projection */
    int32_t lm_head_format;    /* AARH_W_F32 or AARH_W_BF16: tied embedding / LM head storage */
    int32_t kv_format;         /* AARH_KV_* */
    int32_t max_batch;         /* KV-cache sequence slots */
    int32_t max_rows;          /* max rows (sequences x tokens) per forward call, <= 512 */
    int32_t untied_lm_head;    /* 0: LM head tied to the embedding (tie_embeddings = true);
                                  1: its own lm_head.weight [vocab][hidden] in lm_head_format,
                                  the last tensor id, shared by the MTP heads' output
                                  projection (model.rs:239-262) */
} aarh_model_config;

/* Sampler (inference/src/sampler.rs:14-65); probabilities as filtered_probs (:226-278). */
typedef struct {
    int32_t greedy;    /* 1 = Sampler::Greedy */
    float temperature; /* TopKTopP temperature (<= f32::EPSILON behaves greedy) */
    int32_t top_k;     /* <= 0: none (Option::None); >= vocab: keeps every token */
    float top_p;       /* in [0, 1]; 0 or 1: none (top_p.filter(0 < p < 1)) */
} aarh_sampler;

/* SpeculativeStats (inference/src/speculative.rs:41-90). */
typedef struct {
    int32_t rounds, draft_tokens_proposed, draft_tokens_accepted, draft_tokens_rejected;
    int32_t target_decode_forwards, draft_decode_forwards, mtp_head_forwards;
} aarh_spec_stats;

/* --- context (replaces InferenceEngine::from_paths_with_dtype, inference/src/engine.rs:226-244) --- */
int aarh_create(int device, const aarh_model_config *cfg, aarh_ctx **out);
void aarh_destroy(aarh_ctx *ctx);
const char *aarh_last_error(const aarh_ctx *ctx);
void *aarh_stream(aarh_ctx *ctx); /* the context's hipStream_t */
int aarh_sync(aarh_ctx *ctx);

/* --- weights: checkpoint tensors by reference name/order (model/src/model.rs:82-279) --- */
int aarh_num_tensors(const aarh_ctx *ctx);
int aarh_tensor_info(const aarh_ctx *ctx, int id, char *name, int name_cap, int64_t *rows,
                     int64_t *cols, int32_t *kind);
/* f32 host values, quantised on device per the configured format
   (quantise_affine_i4 int4.rs:7-41 / fake_quant_symmetric qat.rs:155-169). */
int aarh_load_tensor_f32(aarh_ctx *ctx, int id, const float *host, int64_t numel);
/* PackedInt4Tensor (types.rs:79-90) with fp16 scale/zero per 128-group, row-major. */
int aarh_load_tensor_int4(aarh_ctx *ctx, int id, const uint8_t *packed, const uint16_t *scales_f16,
                          const uint16_t *zeros_f16, int64_t rows, int64_t cols, int32_t group);
/* A PackedInt4Tensor as the quant crate defines it (quant/src/types.rs:79-90: shape,
   group_size, data = packed nibbles over the flattened row-major tensor, low nibble first,
   int4.rs:45-53; f32 scales and zeros per group, value = (q - zero) * scale,
   dequantise_packed_i4_to_vec int4.rs:70-91).  shape must be the tensor's [rows, cols].
   Errors as the reference: CONFIG for group_size 0, SHAPE for a group count other than
   ceil(numel / group_size) or too few data bytes.  The device keeps one fp16 scale and
   one fp16 zero per 128 columns of a row, so the load needs group_size and cols to be
   multiples of 128 (UNSUPPORTED otherwise), each scale is rounded to the nearest fp16
   value (ties to even; UNSUPPORTED when that is infinite) and each zero must be an
   integer with |zero| < 1024 (kept exactly).  The device then multiplies by
   (q - zero) * fp16(scale): equal to the reference's value whenever the scale is an fp16
   value, within 2^-11 of it relatively for normal-range scales otherwise. */
int aarh_load_tensor_packed_i4(aarh_ctx *ctx, int id, const int64_t *shape, int32_t ndims,
                               int64_t group_size, const uint8_t *data, int64_t data_len,
                               const float *scales, const float *zeros, int64_t n_groups);
/* The conversion aarh_load_tensor_packed_i4 applies, without a context or a GPU: fills
   scales_f16 / zeros_f16 [rows][cols / 128] (rows = product of all but the last dim) with
   the fp16 parameters of each 128-column device group; same checks and errors (message
   in aarh_host_last_error). */
int aarh_packed_i4_params(const int64_t *shape, int32_t ndims, int64_t group_size, int64_t data_len,
                          const float *scales, const float *zeros, int64_t n_groups,
                          uint16_t *scales_f16, uint16_t *zeros_f16);
/* Per-row INT8 codes + f32 row scales (I8QuantizedTensor semantics per channel). */
int aarh_load_tensor_int8(aarh_ctx *ctx, int id, const int8_t *codes, const float *scales,
                          int64_t rows, int64_t cols);
/* The configuration the context was created with. */
int aarh_get_config(const aarh_ctx *ctx, aarh_model_config *out);

/* --- checkpoints (host readers; tensors decoded to f32 as the reference decodes them, then
   quantised on device into the context's formats like aarh_load_tensor_f32) ---
   GGUF v1 (load_gguf_tensors, weights/src/gguf.rs:91-241): F32, Q8_0 (per-tensor absmax,
   dequant.rs:7-16) and Q4_K_M (gguf_quant.rs:37-49, custom f16 at :51-112).  The file's
   config (config.rs:734-776) must match the context's shape, rope_theta and norm_eps and its
   tie_embeddings must match untied_lm_head (CONFIG otherwise; a config without it is a
   CHECKPOINT error, as serde requires the field); moe / attention_schedule / dsa_config are
   UNSUPPORTED here (aarh_lat_load_gguf takes MLA + MoE files).  The file's rope_scaling (or
   its absence) is applied as aarh_set_rope_scaling does, before any tensor is read.
   safetensors (load_model_with_dtype, weights/src/lib.rs:68-79): F32, F16 and BF16 values.
   Every context tensor must be present with its checkpoint shape (norms 1-D); other tensors
   are ignored, as VarBuilder reads by name.  *out_loaded (optional) = tensors loaded. */
int aarh_load_gguf(aarh_ctx *ctx, const char *path, int32_t *out_loaded);
int aarh_load_safetensors(aarh_ctx *ctx, const char *path, int32_t *out_loaded);
/* Fills the model-shape fields of *out (vocab_size .. max_seq_len, rope_theta, norm_eps,
   num_future_tokens from mtp, untied_lm_head from tie_embeddings) from a GGUF file's config; formats and sizing are left to
   the caller (the file is what from_paths reads its config from, engine.rs:226-244). */
int aarh_gguf_config(const char *path, aarh_model_config *out);
/* Decodes one GGUF tensor to f32 on the host (no context, no GPU).  out may be NULL to query
   numel/ndims/shape (shape holds up to 8 dims)/encoding (0 F32, 1 Q8_0, 2 Q4_K_M). */
int aarh_gguf_read_tensor(const char *path, const char *name, float *out, int64_t cap,
                          int64_t *out_numel, int32_t *out_ndims, int64_t *out_shape,
                          int32_t *out_encoding);
/* Decodes one safetensors tensor (F32 / F16 / BF16) to f32 on the host (no context, no GPU). */
int aarh_safetensors_read_tensor(const char *path, const char *name, float *out, int64_t cap,
                                 int64_t *out_numel, int32_t *out_ndims, int64_t *out_shape);
/* Message of the last failure of a context-free call on this thread. */
const char *aarh_host_last_error(void);

/* Random-init model generated on device: N(0, std^2) linears/embedding, norms 1.0. */
int aarh_init_synthetic(aarh_ctx *ctx, uint64_t seed, float std);

/* --- KV cache (inference/src/kvcache.rs:22-69; rollback by index, nn/src/kvcache.rs:301-304) --- */
int aarh_kv_reset(aarh_ctx *ctx, int slot);
int aarh_kv_len(const aarh_ctx *ctx, int slot, int32_t *out_len);
int aarh_kv_rollback(aarh_ctx *ctx, int slot, int32_t new_len);
int aarh_kv_fill_synthetic(aarh_ctx *ctx, int slot, int32_t len, uint64_t seed);

/* --- model forward (AarambhModel::forward_with_cache_output, model.rs:529-587) ---
   ids [nseq][S] for cache slots slots[nseq] at offsets[nseq] (offset <= cached length;
   a smaller offset rewinds that slot first).  Logits [nseq][S][vocab] and final normed
   hidden states [nseq][S][hidden] are copied to host when the pointers are non-null. */
int aarh_forward(aarh_ctx *ctx, const uint32_t *ids, const int32_t *slots, const int32_t *offsets,
                 int nseq, int S, float *logits_out, float *hidden_out);
/* Device pointers of the last forward's outputs (valid until the next call). */
const float *aarh_last_logits_device(const aarh_ctx *ctx);
const float *aarh_last_hidden_device(const aarh_ctx *ctx);

/* --- MTP head (AarambhModel::forward_mtp_head, model.rs:783-817) ---
   anchor [nseq][hidden] (final normed hidden of the anchor position), ids [nseq][head+1]. */
int aarh_mtp_head(aarh_ctx *ctx, int head, const float *anchor, const uint32_t *ids, int nseq,
                  float *logits_out);

/* --- acceptance (accept_proposal / residual_distribution / sample_probabilities,
   inference/src/speculative.rs:755-793, sampler.rs:102-347), all DEVICE pointers:
   target [B][target_rows][V], draft [B][K][V], draft_tokens [B][K], n_proposals [B] or NULL,
   seeds/word_offsets [B] (StdRng::seed_from_u64 keystream position) or uniforms [B][K+1].
   bonus = 1 samples from target row n_proposals when every proposal is accepted
   (external-draft round); bonus = 0 is the MTP round.  Outputs [B]: accepted count,
   replacement/bonus token (-1 none), near-tie flags, uniforms consumed, status (0 ok,
   1 zero-mass residual or invalid distribution).  stream: hipStream_t or NULL (context stream).
   Any vocabulary size; top-k / top-p apply as in filtered_probs. */
int aarh_accept_sample(aarh_ctx *ctx, const float *target, int target_rows, const float *draft,
                       const uint32_t *draft_tokens, const int32_t *n_proposals, int B, int K, int V,
                       int bonus, const aarh_sampler *sampler, const uint64_t *seeds,
                       const uint64_t *word_offsets, const float *uniforms, int32_t *accept_len,
                       int32_t *token, uint32_t *flags, int32_t *draws, int32_t *status, void *stream);

/* aarh_accept_sample without any allocation.  No counterpart in the reference: it is for
   callers that cannot allocate device memory (HIP graph capture, serving loops that forbid
   hipMalloc).  Same arguments and results as aarh_accept_sample; its scratch (row statistics,
   arrival counters) is a statically allocated per-GPU block of the library holding at most
   1024 sequences and 4096 logits rows (B * (target_rows + K)); larger calls fail with
   AARH_ERR_SHAPE.  Every call on one GPU shares that block: calls that overlap on one GPU
   (other streams, other threads, other contexts) race. */
int aarh_accept_sample_static(aarh_ctx *ctx, const float *target, int target_rows, const float *draft,
                              const uint32_t *draft_tokens, const int32_t *n_proposals, int B, int K, int V,
                              int bonus, const aarh_sampler *sampler, const uint64_t *seeds,
                              const uint64_t *word_offsets, const float *uniforms, int32_t *accept_len,
                              int32_t *token, uint32_t *flags, int32_t *draws, int32_t *status, void *stream);

/* --- engine (MtpSpeculativeEngine::generate_with_callback, inference/src/mtp_speculative.rs:86-336)
   for nseq independent requests run in lock-step rounds on slots 0..nseq-1.
   prompts [nseq][prompt_len]; out_tokens [nseq][max_new_tokens]. */
int aarh_mtp_generate(aarh_ctx *ctx, const uint32_t *prompts, int nseq, int prompt_len,
                      int max_new_tokens, int num_draft_tokens, const aarh_sampler *sampler,
                      const uint64_t *seeds, uint32_t *out_tokens, int32_t *out_len,
                      int32_t *finish_reason, aarh_spec_stats *stats);

/* The same engine as a session, one call per batch of rounds (serving / benchmarking).
   begin: prefills prompts [nseq][prompt_len] on top of `cached_len` tokens already held by
   each slot's KV cache (0 = fresh request; the context limit counts cached + prompt tokens).
   step: runs up to max_rounds speculative rounds (mtp_speculative.rs:161-322).
   result: committed tokens [nseq][out_cap], lengths, finish reasons, SpeculativeStats. */
typedef struct aarh_session aarh_session;
int aarh_session_begin(aarh_ctx *ctx, const uint32_t *prompts, int nseq, int prompt_len, int cached_len,
                       int max_new_tokens, int num_draft_tokens, const aarh_sampler *sampler,
                       const uint64_t *seeds, aarh_session **out);
int aarh_session_step(aarh_session *session, int max_rounds, int32_t *all_done);
int aarh_session_result(aarh_session *session, uint32_t *out_tokens, int32_t out_cap, int32_t *out_len,
                        int32_t *finish_reason, aarh_spec_stats *stats);
/* Top AARH_TOP_CANDIDATES candidates (token id, probability) of every committed token, from the
   target distribution of its position: Sampler::top_candidates_from_probabilities
   (inference/src/sampler.rs:188-208, engine.rs:70 top_candidates = 5; GenerationStep.candidates
   engine.rs:95-110).  ids/probs [nseq][out_cap][AARH_TOP_CANDIDATES], host memory. */
int aarh_session_candidates(aarh_session *session, uint32_t *ids, float *probs, int32_t out_cap);
/* Keystream position (StdRng word offset) of each request [nseq]: the next uniform a
   request draws is word `offset` of StdRng::seed_from_u64(seed).  The reference's
   Sampler owns its StdRng and keeps it across generate calls (sampler.rs:39-65,
   157-162); set restores a saved position before the next step (resuming a request). */
int aarh_session_rng_offsets(aarh_session *session, uint64_t *out);
int aarh_session_set_rng_offsets(aarh_session *session, const uint64_t *offsets);
void aarh_session_end(aarh_session *session);

/* Continuous batching of speculative requests: the serving worker's loop
   (serve/src/batching.rs:324-445: admit while active < max_batch_size, advance, drop
   finished or cancelled requests, then one batched decode) with its batched decode
   (InferenceEngine::decode_sessions, inference/src/engine.rs:323-355) replaced by MTP
   speculative rounds.  open: a session of `capacity` rows (<= max_batch), all free.
   admit: a free row takes a request (prompt of its own length, its own token budget
   and sampler seed): prepare_session_with_chunk_size (engine.rs:271-317) prefills the
   prompt from position 0 of the row's KV slot in forwards of at most prefill_chunk
   tokens; errors as there (SHAPE: prompt_len >= max_seq_len; CONFIG: chunk 0).
   aarh_session_step then runs rounds over every generating row; aarh_session_result /
   _candidates report every row (free rows: length 0).  retire: the row's request
   leaves (completed or cancelled) and the row and its slot are free again.
   rows: per row 0 = free, 1 = generating, 2 = finished (result ready, not retired).
   Requests share the session's sampler settings (temperature, top-k, top-p).  Row b
   uses KV slot b: the session owns slots 0..capacity-1, and a free row's slot keeps
   no cache (rounds write padding rows at its position 0). */
int aarh_session_open(aarh_ctx *ctx, int capacity, int num_draft_tokens, const aarh_sampler *sampler,
                      aarh_session **out);
int aarh_session_admit(aarh_session *session, int row, const uint32_t *prompt, int prompt_len,
                       int max_new_tokens, uint64_t seed, int prefill_chunk);
int aarh_session_retire(aarh_session *session, int row);
int aarh_session_rows(aarh_session *session, int32_t *state);

/* --- external-draft engine (SpeculativeEngine::generate_with_callback,
   inference/src/speculative.rs:175-516; constructor checks :101-122) ---
   target and draft are contexts of two models with the same vocabulary on one device;
   both hold nseq requests on slots 0..nseq-1 (prefilled here from fresh caches).  Each
   round the draft proposes up to num_draft_tokens (1..31) tokens autoregressively, the
   target verifies [pending?] + proposals in one forward, the fused acceptance kernel
   tests them in order and samples the replacement (rejection) or bonus token (all
   accepted), both caches roll back by index and replay the accepted prefix.  The
   context limit is the smaller of the two models' max_seq_len.  Outputs as for
   aarh_mtp_generate, plus (when non-NULL) the committed tokens' top candidates
   [nseq][max_new_tokens][AARH_TOP_CANDIDATES] as for aarh_session_candidates. */
int aarh_spec_generate(aarh_ctx *target, aarh_ctx *draft, const uint32_t *prompts, int nseq,
                       int prompt_len, int max_new_tokens, int num_draft_tokens,
                       const aarh_sampler *sampler, const uint64_t *seeds, uint32_t *out_tokens,
                       int32_t *out_len, int32_t *finish_reason, aarh_spec_stats *stats,
                       uint32_t *out_cand_ids, float *out_cand_probs);

/* The external-draft engine as a session, one call per batch of rounds
   (speculative.rs:175-516, as aarh_spec_generate, which is begin + step until done +
   result + candidates + end).  begin: the constructor checks and both prefills
   (speculative.rs:236-247); step: up to max_rounds rounds (:251-508); result /
   candidates: committed tokens, finish reasons, SpeculativeStats and top candidates so
   far (out_cap tokens per request).  rng_offsets / set_rng_offsets: the keystream
   position (StdRng word offset) of each request's sampler, as for aarh_session_*. */
typedef struct aarh_spec_session aarh_spec_session;
int aarh_spec_session_begin(aarh_ctx *target, aarh_ctx *draft, const uint32_t *prompts, int nseq,
                            int prompt_len, int max_new_tokens, int num_draft_tokens,
                            const aarh_sampler *sampler, const uint64_t *seeds, aarh_spec_session **out);
int aarh_spec_session_step(aarh_spec_session *session, int max_rounds, int32_t *all_done);
int aarh_spec_session_result(aarh_spec_session *session, uint32_t *out_tokens, int32_t out_cap,
                             int32_t *out_len, int32_t *finish_reason, aarh_spec_stats *stats);
int aarh_spec_session_candidates(aarh_spec_session *session, uint32_t *ids, float *probs, int32_t out_cap);
int aarh_spec_session_rng_offsets(aarh_spec_session *session, uint64_t *out);
int aarh_spec_session_set_rng_offsets(aarh_spec_session *session, const uint64_t *offsets);
void aarh_spec_session_end(aarh_spec_session *session);

/* --- Sampler::top_candidates_from_probabilities (sampler.rs:188-208) of each row's sampling
   distribution (Sampler::probabilities: greedy one-hot at the argmax, else softmax at T):
   the n <= AARH_TOP_CANDIDATES largest probabilities, ties in ascending token order.
   logits [rows][V], ids/probs [rows][n]: DEVICE pointers; stream as for aarh_accept_sample. */
int aarh_top_candidates(aarh_ctx *ctx, const float *logits, int rows, int V, const aarh_sampler *sampler,
                        int n, uint32_t *ids, float *probs, void *stream);

/* --- RoPE scaling (RopeScalingConfig, core/src/config.rs:22-35; applied by
   inverse_frequencies_for_config, nn/src/rope_scaling.rs:24-92, to the transformer's RoPE
   cache, nn/src/rope.rs:17-28).  Rebuilds the context's cos / sin tables in place:
   linear divides the base inverse frequencies by factor, NTK raises theta by
   factor^(hd / (hd - 2)), YaRN blends the extrapolated and factor-interpolated frequency by a
   linear ramp over the beta_fast / beta_slow correction range at original_max_seq_len; every
   method multiplies cos and sin by attn_factor.  NULL or method AARH_ROPE_NONE restores the
   unscaled tables.  Validation follows RopeScalingConfig::validate (config.rs:52-96):
   AARH_ERR_CONFIG with its message, tables unchanged.  Call between forwards (it waits for
   the context's stream); latent contexts are unaffected, since MLA keeps an unscaled RoPE
   cache of its own (model.rs:1107-1116). --- */
enum { AARH_ROPE_NONE = 0, AARH_ROPE_YARN = 1, AARH_ROPE_NTK = 2, AARH_ROPE_LINEAR = 3 };
typedef struct aarh_rope_scaling {
    int32_t method;               /* AARH_ROPE_* */
    int32_t original_max_seq_len; /* base model's training context */
    double factor;                /* context extension factor, > 1 */
    double beta_fast;             /* YaRN high-frequency correction boundary */
    double beta_slow;             /* YaRN low-frequency correction boundary */
    double attn_factor;           /* cos / sin multiplier, > 0 */
} aarh_rope_scaling;
int aarh_set_rope_scaling(aarh_ctx *ctx, const aarh_rope_scaling *scaling);
/* A GGUF file's config rope_scaling (serde defaults per field: method yarn, factor 1,
   original_max_seq_len 0, beta_fast 32, beta_slow 1, attn_factor 1; method AARH_ROPE_NONE
   when absent).  Values are not validated here; aarh_set_rope_scaling does that. */
int aarh_gguf_rope_scaling(const char *path, aarh_rope_scaling *out);

/* --- launch mode: repeated verify-forward shapes replay a captured HIP graph (default on;
   0 launches every kernel from the host each call).  Results are identical either way. --- */
int aarh_set_graphs(aarh_ctx *ctx, int enable);

/* --- MTP rejection replay schedule.  AARH_REPLAY_REPLACEMENT (default): the verify forward
   already wrote the accepted proposals' K / V at their positions, so only the replacement
   token is forwarded.  AARH_REPLAY_REFERENCE: restore to the round's base and forward
   proposals[..i] + replacement as mtp_speculative.rs:284-313 does.  Both give the same
   function; they differ only in rounding (which rows are computed together). --- */
enum { AARH_REPLAY_REPLACEMENT = 0, AARH_REPLAY_REFERENCE = 1 };
int aarh_set_replay_schedule(aarh_ctx *ctx, int schedule);

/* --- measurement: per-kernel-class timing of the context's launches (HIP events recorded
   at each kernel dispatch's own start and end; graph replay is off while enabled) --- */
enum { AARH_PROF_GEMV_QKV = 0, AARH_PROF_GEMV_WO = 1, AARH_PROF_GEMV_GATEUP = 2,
       AARH_PROF_GEMV_DOWN = 3, AARH_PROF_GEMV_LMHEAD = 4, AARH_PROF_ATTENTION = 5,
       AARH_PROF_ACCEPT = 6, AARH_PROF_OTHER = 7, AARH_PROF_COUNT = 8 };
int aarh_prof_enable(aarh_ctx *ctx, int enable);
int aarh_prof_get(aarh_ctx *ctx, int cls, double *total_ms, double *alg_bytes, int64_t *launches);

/* ===================================================================================
 * Latent-attention MoE decoder (benchmark config 5): blocks of multi-head latent
 * attention (nn/src/mla.rs:300-489, built by model/src/model.rs:1094-1156) and a
 * fine-grained MoE FFN with top-k routing and shared experts (nn/src/moe.rs:127-406).
 * A separate context type with the same conventions as aarh_ctx; its cache holds the
 * normalised KV latent c_kv and the rotated shared key k_rope per token (fp16).
 * =================================================================================== */
typedef struct aarh_lat_ctx aarh_lat_ctx;

/* MlaConfig (core/src/config.rs MLA fields) + MoeConfig (fine experts, shared experts)
   + formats + device sizing. */
typedef struct {
    int32_t vocab_size, hidden_dim, n_layers, n_heads, max_seq_len;
    float rope_theta, norm_eps;
    int32_t latent_dim, rope_dim, nope_dim, v_dim; /* (512, 64) or (128, 32) latent/rope widths */
    int32_t n_experts, top_k, expert_dim, n_shared;
    int32_t expert_format;  /* AARH_W_BF16 / INT8_ROW / INT4_G128: routed + shared experts */
    int32_t attn_format;    /* AARH_W_*: MLA projections and the router */
    int32_t lm_head_format; /* AARH_W_F32 or AARH_W_BF16: the LM head (and the embedding) */
    int32_t kv_format;      /* AARH_KV_F16 (the latent cache is fp16) */
    int32_t max_batch;      /* cache sequence slots */
    int32_t max_rows;       /* max rows (sequences x tokens) per forward, <= 256 */
    int32_t untied_lm_head; /* 0: the LM head reads the embedding (tie_embeddings); 1: its own
                               lm_head.weight [vocab][hidden] after final_norm
                               (LmHead::untied_with_qat, model.rs:239-248) */
} aarh_lat_config;

/* Context + weights (checkpoint names and order of the latent decoder, as
   AarambhModel::named_tensors writes them, model.rs:1053-1054, mla.rs:383-393,
   model.rs:944-1000: embedding, per layer blocks.{l}.norm1, blocks.{l}.mla.{q_proj,
   kv_a_proj, kv_a_norm, up_k, up_v, k_rope_proj, o_proj}, norm2, ffn.router,
   ffn.experts.{e}.{w_gate,w_up,w_down}, ffn.shared_experts.{s}.{...}, then final_norm, then
   lm_head when untied_lm_head). */
int aarh_lat_create(int device, const aarh_lat_config *cfg, aarh_lat_ctx **out);
void aarh_lat_destroy(aarh_lat_ctx *ctx);
const char *aarh_lat_last_error(const aarh_lat_ctx *ctx);
int aarh_lat_num_tensors(const aarh_lat_ctx *ctx);
int aarh_lat_tensor_info(const aarh_lat_ctx *ctx, int id, char *name, int name_cap, int64_t *rows,
                         int64_t *cols, int32_t *kind);
int aarh_lat_load_tensor_f32(aarh_lat_ctx *ctx, int id, const float *host, int64_t numel);
/* The configuration the latent context was created with. */
int aarh_lat_get_config(const aarh_lat_ctx *ctx, aarh_lat_config *out);
/* Checkpoints of an MLA + MoE model (AarambhModel::new over the checkpoint's VarBuilder,
   model.rs:82-279: block_vb.pp("mla") per MLA layer, ffn.router / ffn.experts.{e} /
   ffn.shared_experts.{s} per MoE layer), read and decoded as aarh_load_gguf /
   aarh_load_safetensors do.  GGUF: the file's config is validated as
   AarambhModel::validate_config does (model.rs:281-344: MoeConfig, the attention schedule
   with its MLA and Gated DeltaNet settings, RopeScalingConfig, dsa_config; CONFIG with the
   reference's message), then must describe what a latent context holds -- MLA in every
   layer (attention_schedule.mla_layers = 0..n_layers), MoE in every layer
   (moe.every_n_layers = 1), UNSUPPORTED otherwise -- and match the context's shape and
   its untied_lm_head (tie_embeddings false: lm_head.weight is read; CONFIG otherwise).  rope_scaling is validated but changes nothing, since MLA keeps
   an unscaled RoPE cache (model.rs:1107-1116); mtp heads are not part of the latent
   context and are not read.  Every context tensor must be present with its shape. */
int aarh_lat_load_gguf(aarh_lat_ctx *ctx, const char *path, int32_t *out_loaded);
int aarh_lat_load_safetensors(aarh_lat_ctx *ctx, const char *path, int32_t *out_loaded);
/* A GGUF file's config resolved into the latent shape fields of *out (vocab_size,
   hidden_dim, n_layers, n_heads = resolved MLA heads, max_seq_len, rope_theta, norm_eps,
   latent/rope/nope/v widths from MlaConfig::resolve, n_experts = num_experts x
   fine_grained_factor, top_k, expert_dim = expert_ffn_dim / fine_grained_factor,
   n_shared = num_shared_experts, untied_lm_head = !tie_embeddings); same checks and errors as aarh_lat_load_gguf's config
   step, message in aarh_host_last_error.  Formats and sizing are left to the caller. */
int aarh_lat_gguf_config(const char *path, aarh_lat_config *out);
/* A PackedInt4Tensor (quant/src/types.rs:79-90) into an INT4 g128 tensor of the latent
   decoder (experts in expert_format, MLA projections and the router in attn_format);
   same rules, rounding and errors as aarh_load_tensor_packed_i4. */
int aarh_lat_load_tensor_packed_i4(aarh_lat_ctx *ctx, int id, const int64_t *shape, int32_t ndims,
                                   int64_t group_size, const uint8_t *data, int64_t data_len,
                                   const float *scales, const float *zeros, int64_t n_groups);
/* Random init on device: tensor id i ~ N(0, std^2) (router N(0, 1/hidden_dim)), norms 1. */
int aarh_lat_init_synthetic(aarh_lat_ctx *ctx, uint64_t seed, float std);

/* Latent cache per slot (MlaKvCache; rollback by index like nn/src/kvcache.rs:301-304). */
int aarh_lat_kv_len(const aarh_lat_ctx *ctx, int slot, int32_t *out_len);
int aarh_lat_kv_rollback(aarh_lat_ctx *ctx, int slot, int32_t new_len);
int aarh_lat_kv_fill_synthetic(aarh_lat_ctx *ctx, int slot, int32_t len, uint64_t seed);

/* Verify forward (as aarh_forward): ids [nseq][S] on slots at offsets; logits
   [nseq][S][vocab], final normed hidden [nseq][S][hidden] when non-null. */
int aarh_lat_forward(aarh_lat_ctx *ctx, const uint32_t *ids, const int32_t *slots, const int32_t *offsets,
                     int nseq, int S, float *logits_out, float *hidden_out);
/* Of the last forward: per row, the smallest gap between the k-th and (k+1)-th router
   logit over all layers ([nseq*S]; a near-tie may route differently from an f32 CPU
   path), and the rows routed to each expert per layer ([n_layers][n_experts + n_shared]). */
int aarh_lat_router_gaps(aarh_lat_ctx *ctx, float *out);
int aarh_lat_expert_counts(aarh_lat_ctx *ctx, int32_t *out);

/* Per-class timing as aarh_prof_*: QKV = fused q / kv_a / k_rope projection, WO =
   o_proj, GATEUP = router + routing + expert gate/up, DOWN = expert down + combine,
   ATTENTION = q absorption, cache append, latent attention, up_v, LMHEAD. */
int aarh_lat_prof_enable(aarh_lat_ctx *ctx, int enable);
int aarh_lat_prof_get(aarh_lat_ctx *ctx, int cls, double *total_ms, double *alg_bytes, int64_t *launches);

#ifdef __cplusplus
}
#endif
#endif
