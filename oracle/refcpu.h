/*
 * refcpu: CPU oracle for the speculative-decoding verify path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library restates the reference CPU path of
 * aarambh-studio (Rust, /root/reference) in plain C so that the HIP library can
 * be checked against it.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library never links or calls it.
 *
 * Every function cites the reference file:line it restates.  Parity status of
 * each part (what pins it) is listed in the header comment of refcpu.c.
 */
#ifndef AARAMBH_REFCPU_H
#define AARAMBH_REFCPU_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes mirror AarambhError variants (core/src/error.rs:5-33). */
enum { REF_OK = 0, REF_ERR_CONFIG = 1, REF_ERR_SHAPE = 2, REF_ERR_UNSUPPORTED = 3 };

/* ---------------- RNG: rand 0.8 StdRng = ChaCha12 (rand_chacha 0.3.1) ---------------- */
typedef struct {
    uint32_t key[8];
    uint64_t pos;          /* index of the next keystream word */
    uint64_t cached_block; /* block index held in buf, or UINT64_MAX */
    uint32_t buf[16];
} ref_rng;

void ref_chacha_core(const uint32_t in[16], int rounds, uint32_t out[16]);
uint32_t ref_pcg32_xsh_rr(uint64_t state);
void ref_rng_seed_u64(ref_rng *r, uint64_t seed);
void ref_rng_set_pos(ref_rng *r, uint64_t pos);
uint32_t ref_rng_next_u32(ref_rng *r);
float ref_rng_next_f32(ref_rng *r);
float ref_rng_word_f32(uint64_t seed, uint64_t word_index);

/* ---------------- Sampler (inference/src/sampler.rs) ---------------- */
typedef struct {
    int32_t greedy;      /* 1 = Sampler::Greedy */
    float temperature;   /* TopKTopP temperature */
    int32_t top_k;       /* 0 = None */
    float top_p;         /* outside (0,1) = None */
} ref_sampler;

int ref_is_deterministic(const ref_sampler *s);
int64_t ref_argmax(const float *v, int64_t n);
int ref_probabilities(const ref_sampler *s, const float *logits, int64_t n, float *out);
int ref_validate_probabilities(const float *p, int64_t n);
int ref_sample_probabilities(const ref_sampler *s, ref_rng *rng, const float *p, int64_t n,
                             uint32_t *out_token, float *out_draw, float *out_cdf_margin);
int ref_accept_proposal(const ref_sampler *s, ref_rng *rng, uint32_t token, const float *draft,
                        const float *target, int64_t n, int *accepted, float *out_ratio,
                        float *out_draw, int *drew);
int ref_residual(const float *target, const float *draft, int64_t n, float *out);

/* Batched acceptance: B independent sequences, each one reference round. */
typedef struct {
    int32_t accept_len;   /* accepted proposals */
    int32_t token;        /* replacement (on rejection) or bonus token, -1 if none */
    uint32_t flags;       /* REF_FLAG_* near-tie markers */
    int32_t draws;        /* uniforms consumed */
    float ratio_margin;   /* min |p/q - u| over tests made (inf if none) */
    float cdf_margin;     /* |u - cdf| distance at the final sample (inf if none) */
} ref_accept_result;

enum { REF_FLAG_RATIO_NEAR = 1u, REF_FLAG_CDF_NEAR = 2u, REF_FLAG_ARGMAX_NEAR = 4u, REF_FLAG_TOPP_NEAR = 8u };

/* Margins of the last ref_probabilities call on this thread: top-p cumulative vs top_p
   at the crossing, and the k-th vs (k+1)-th ranked logit gap (INFINITY when unused). */
float ref_last_topp_margin(void);
float ref_last_topk_gap(void);

int ref_accept_batch(int B, int K, int64_t V, const float *target, int target_rows,
                     const float *draft, const uint32_t *draft_tokens, const int32_t *n_proposals,
                     int bonus, const ref_sampler *s, const uint64_t *seeds,
                     const uint64_t *word_offsets, const float *uniforms,
                     ref_accept_result *out);

/* ---------------- Numeric formats and quantisation (quant/src) ---------------- */
uint16_t ref_f32_to_f16(float x);
float ref_f16_to_f32(uint16_t h);
uint16_t ref_f32_to_bf16(float x);
float ref_bf16_to_f32(uint16_t h);
int ref_quantise_i4(const float *w, int64_t n, int64_t group, uint8_t *packed, float *scales,
                    float *zeros);
int ref_dequantise_i4(const uint8_t *packed, int64_t n, int64_t group, const float *scales,
                      const float *zeros, float *out);
int ref_quantise_i4_f16(const float *w, int64_t n, int64_t group, uint8_t *packed,
                        uint16_t *scales_h, uint16_t *zeros_h);
int ref_dequantise_i4_f16(const uint8_t *packed, int64_t n, int64_t group,
                          const uint16_t *scales_h, const uint16_t *zeros_h, float *out);
int ref_quantise_i8_rows(const float *w, int64_t rows, int64_t cols, int8_t *codes, float *scales);
int ref_quantise_kv_row(const float *x, int64_t n, int8_t *codes, uint16_t *scale_h);

/* ---------------- Synthetic inputs (build-defined, shared with the GPU) ---------------- */
uint64_t ref_splitmix64(uint64_t x);
float ref_synth_normal(uint64_t seed, uint32_t stream, uint64_t index);
void ref_synth_fill(uint64_t seed, uint32_t stream, int64_t n, float std, float *out);
void ref_synth_tokens(uint64_t seed, uint32_t stream, int64_t n, uint32_t vocab, uint32_t *out);

/* ---------------- Model (model/src/model.rs, nn/src/ files) ---------------- */
typedef struct {
    int32_t vocab_size, hidden_dim, ffn_dim, n_layers, n_heads, n_kv_heads, max_seq_len;
    float rope_theta, norm_eps;
    int32_t num_future_tokens; /* MTP horizon; 0 = no MTP heads */
    int32_t weight_format;     /* 0 f32, 1 bf16, 2 int8 per-row, 3 int4 g128 */
    int32_t lm_head_format;    /* 0 f32, 1 bf16 (tied embedding storage) */
    int32_t kv_format;         /* 0 f32, 1 f16, 2 int8 per token per kv-head */
    int32_t untied_lm_head;    /* 1: lm_head.weight (last tensor) instead of the embedding */
} ref_config;

enum { REF_W_F32 = 0, REF_W_BF16 = 1, REF_W_INT8_ROW = 2, REF_W_INT4_G128 = 3 };
enum { REF_KV_F32 = 0, REF_KV_F16 = 1, REF_KV_INT8 = 2 };
enum { REF_T_NORM = 0, REF_T_LINEAR = 1, REF_T_EMBED = 2 };

typedef struct ref_model ref_model;
typedef struct ref_kv ref_kv;

ref_model *ref_model_create(const ref_config *cfg);
/* RoPE scaling (rope_scaling.rs:24-92): method 0 none, 1 yarn, 2 ntk, 3 linear. */
int ref_rope_frequencies(int hd, double theta, int max_seq_len, int method, double factor,
                         int original_max_seq_len, double beta_fast, double beta_slow,
                         double attn_factor, float *inv, float *attn, char *err, int err_cap);
int ref_model_set_rope_scaling(ref_model *m, int method, double factor, int original_max_seq_len,
                               double beta_fast, double beta_slow, double attn_factor, char *err, int err_cap);
void ref_model_free(ref_model *m);
int ref_model_num_tensors(const ref_model *m);
int ref_model_tensor_info(const ref_model *m, int id, char *name, int name_cap, int64_t *rows,
                          int64_t *cols, int32_t *kind);
int ref_model_set_tensor(ref_model *m, int id, const float *raw);
int ref_model_get_tensor(const ref_model *m, int id, float *out);
int ref_model_init_synthetic(ref_model *m, uint64_t seed, float std);

ref_kv *ref_kv_create(const ref_model *m, int capacity);
void ref_kv_free(ref_kv *kv);
int ref_kv_len(const ref_kv *kv);
int ref_kv_truncate(ref_kv *kv, int new_len);
int ref_kv_fill_synthetic(ref_kv *kv, uint64_t seed, int len);

int ref_forward(const ref_model *m, ref_kv *kv, const uint32_t *ids, int S, int offset,
                float *logits, float *hidden, int nthreads);
int ref_forward_layers(const ref_model *m, ref_kv *kv, const uint32_t *ids, int S, int offset,
                       int n_layers, int with_head, float *logits, int nthreads);
int ref_mtp_head(const ref_model *m, int head, const float *anchor, const uint32_t *ids,
                 int n_ids, float *logits, int nthreads);

/* ---------------- Engines (inference/src/mtp_speculative.rs, speculative.rs) ---------------- */
typedef struct {
    int32_t rounds, draft_tokens_proposed, draft_tokens_accepted, draft_tokens_rejected;
    int32_t target_decode_forwards, draft_decode_forwards, mtp_head_forwards;
} ref_spec_stats;

enum { REF_FINISH_MAX_TOKENS = 0, REF_FINISH_EOS = 1, REF_FINISH_CONTEXT_LIMIT = 2 };

/* One engine round (test diagnostics): start state, outcome and decision margins. */
typedef struct {
    uint64_t rng_pos_before;   /* keystream word position when the round starts */
    uint64_t rng_pos_after;
    int32_t committed_before;  /* tokens committed before the round */
    int32_t committed_after;
    int32_t proposed, accepted;
    float prob_margin;         /* min |p/q - u|, |cdf - u| (proposal, residual, bonus draws), top-p margin */
    float logit_gap;           /* min top-2 logit gap (greedy) or top-k boundary gap (sampled) */
} ref_round;
/* Rounds of subsequent ref_mtp_generate / ref_spec_generate calls go to buf[0..cap);
   *count receives the number of rounds run.  buf = NULL turns the trace off. */
void ref_set_round_sink(ref_round *buf, int cap, int *count);

int ref_mtp_generate(const ref_model *m, const uint32_t *prompt, int prompt_len,
                     int max_new_tokens, int num_draft_tokens, const ref_sampler *s,
                     uint64_t seed, int nthreads, uint32_t *out_tokens, int *out_len,
                     int *finish_reason, ref_spec_stats *stats, float *out_min_gap);
int ref_spec_generate(const ref_model *tm, const ref_model *dm, const uint32_t *prompt, int prompt_len,
                      int max_new_tokens, int num_draft_tokens, const ref_sampler *s, uint64_t seed,
                      int nthreads, uint32_t *out_tokens, int *out_len, int *finish_reason,
                      ref_spec_stats *stats, float *out_min_gap);
int ref_plain_generate(const ref_model *m, const uint32_t *prompt, int prompt_len,
                       int max_new_tokens, const ref_sampler *s, uint64_t seed, int nthreads,
                       uint32_t *out_tokens, int *out_len, int *finish_reason);

/* ---------------- Latent-attention MoE decoder (benchmark config 5) ---------------- */
typedef struct {
    int32_t vocab_size, hidden_dim, n_layers, n_heads, max_seq_len;
    float rope_theta, norm_eps;
    int32_t latent_dim, rope_dim, nope_dim, v_dim;   /* MLA (nn/src/mla.rs) */
    int32_t n_experts, top_k, expert_dim, n_shared;  /* routed fine experts, top-k, fine width, shared */
    int32_t expert_format;                           /* routed + shared expert weights (REF_W_*) */
    int32_t attn_format;                             /* MLA projections and the router */
    int32_t lm_head_format;                          /* 0 f32, 1 bf16 */
    int32_t kv_format;                               /* latent cache: REF_KV_F32 or REF_KV_F16 */
    int32_t untied_lm_head;                          /* 1: lm_head.weight after final_norm (model.rs:239-248) */
} ref_lat_config;

typedef struct ref_lat ref_lat;
typedef struct ref_lat_kv ref_lat_kv;
ref_lat *ref_lat_create(const ref_lat_config *cfg);
void ref_lat_free(ref_lat *m);
int ref_lat_num_tensors(const ref_lat *m);
int ref_lat_tensor_info(const ref_lat *m, int id, char *name, int name_cap, int64_t *rows, int64_t *cols,
                        int32_t *kind);
int ref_lat_set_tensor(ref_lat *m, int id, const float *raw);
int ref_lat_get_tensor(const ref_lat *m, int id, float *out);
int ref_lat_init_synthetic(ref_lat *m, uint64_t seed, float std);
ref_lat_kv *ref_lat_kv_create(const ref_lat *m, int capacity);
void ref_lat_kv_free(ref_lat_kv *kv);
int ref_lat_kv_truncate(ref_lat_kv *kv, int new_len);
int ref_lat_kv_fill_synthetic(ref_lat_kv *kv, uint64_t seed, int len);
int ref_lat_forward(const ref_lat *m, ref_lat_kv *kv, const uint32_t *ids, int S, int offset, float *logits,
                    float *hidden, int nthreads);
void ref_topk_gating(const float *logits, int rows, int E, int k, int32_t *idx, float *w);

/* Sampler::top_candidates_from_probabilities (sampler.rs:188-208) and a sink that
   records the 5 candidates of every token the engines commit ([cap][5]; NULL: off). */
void ref_top_candidates(const float *p, int64_t n, int k, uint32_t *ids, float *probs);
void ref_set_candidate_sink(uint32_t *ids, float *probs, int cap);

#ifdef __cplusplus
}
#endif
#endif
