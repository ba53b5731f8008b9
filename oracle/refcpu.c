/*
 * refcpu.c -- CPU oracle for the speculative-decoding verify path.
 *
 * TEST INFRASTRUCTURE ONLY: a plain-C restatement of the reference CPU path of
 * aarambh-studio (/root/reference, Rust).  It is the parity checker for the HIP
 * library and, run multi-threaded, the reported CPU baseline ("port").  The
 * product path never links or calls it.
 *
 * What pins each part (parity status):
 *   RNG (ref_chacha_core, ref_rng_*)     RFC 7539 2.3.2 ChaCha20 block vector and the
 *                                         keystream vector of rand_chacha's own test
 *                                         (tests/test_oracle_rng.py).  The 12-round
 *                                         StdRng stream and seed_from_u64 fill are
 *                                         restated from the published rand_chacha 0.3.1 /
 *                                         rand_core 0.6.4 algorithms: no reference test
 *                                         pins the stream bit-exactly -> "parity
 *                                         unpinned" for the exact StdRng word values.
 *   Sampler / acceptance / residual       Reference KATs speculative.rs:906-919,952-960,
 *                                         sampler.rs:353-420, the 50k-draw distribution
 *                                         test speculative.rs:926-950, brute force over
 *                                         tiny vocabularies.
 *   INT4 / INT8 codecs                    int4.rs:93-121 KATs, exhaustive closed-form
 *                                         checks, round-half-away-from-zero rule.
 *   Forward (norm, RoPE, attention, FFN)  Cached == full forward (model_tests.rs:178-203),
 *                                         attention vs softmax closed form, RoPE norm
 *                                         preservation, numpy restatements of textbook
 *                                         definitions, zero-weight last-index argmax.
 *   MTP engine                            Speculative greedy ids == plain greedy ids
 *                                         (mtp_speculative.rs:438-454), forward counts,
 *                                         context-limit KAT (speculative.rs:1030-1043).
 *
 * Floating-point: compiled with -ffp-contract=off so that every f32 expression
 * rounds like the reference Rust code (which never contracts); fmaf is used only
 * inside dot products, where the reference's gemm crate also uses FMA and parity
 * is a tolerance.
 */
#include "refcpu.h"

#include <float.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ======================================================================== */
/* RNG: rand 0.8 StdRng = rand_chacha 0.3.1 ChaCha12Rng, seeded through     */
/* rand_core 0.6.4 SeedableRng::seed_from_u64.  Used by sampler.rs:55-58,   */
/* draw_uniform sampler.rs:157-162 and sample_from_probs sampler.rs:337-347. */
/* ======================================================================== */

#define ROTL32(v, n) (((v) << (n)) | ((v) >> (32 - (n))))
#define QUARTER(a, b, c, d)                                                                      \
    do {                                                                                         \
        a += b; d ^= a; d = ROTL32(d, 16);                                                       \
        c += d; b ^= c; b = ROTL32(b, 12);                                                       \
        a += b; d ^= a; d = ROTL32(d, 8);                                                        \
        c += d; b ^= c; b = ROTL32(b, 7);                                                        \
    } while (0)

/* ChaCha block function (RFC 7539 section 2.3) with a configurable round count. */
void ref_chacha_core(const uint32_t in[16], int rounds, uint32_t out[16]) {
    uint32_t x[16];
    memcpy(x, in, sizeof(x));
    for (int r = 0; r < rounds; r += 2) {
        QUARTER(x[0], x[4], x[8], x[12]);
        QUARTER(x[1], x[5], x[9], x[13]);
        QUARTER(x[2], x[6], x[10], x[14]);
        QUARTER(x[3], x[7], x[11], x[15]);
        QUARTER(x[0], x[5], x[10], x[15]);
        QUARTER(x[1], x[6], x[11], x[12]);
        QUARTER(x[2], x[7], x[8], x[13]);
        QUARTER(x[3], x[4], x[9], x[14]);
    }
    for (int i = 0; i < 16; i++) out[i] = x[i] + in[i];
}

/* PCG XSH-RR output function (O'Neill 2014). */
uint32_t ref_pcg32_xsh_rr(uint64_t state) {
    uint32_t xorshifted = (uint32_t)(((state >> 18) ^ state) >> 27);
    uint32_t rot = (uint32_t)(state >> 59);
    return (xorshifted >> rot) | (xorshifted << ((32 - rot) & 31));
}

/* seed_from_u64: advance a PCG32 state first, then emit; 8 words fill the 32-byte key. */
void ref_rng_seed_u64(ref_rng *r, uint64_t state) {
    const uint64_t mul = 6364136223846793005ull;
    const uint64_t inc = 11634580027462260723ull;
    for (int i = 0; i < 8; i++) {
        state = state * mul + inc;
        r->key[i] = ref_pcg32_xsh_rr(state);
    }
    r->pos = 0;
    r->cached_block = UINT64_MAX;
}

void ref_rng_set_pos(ref_rng *r, uint64_t pos) { r->pos = pos; }

static void rng_block(const uint32_t key[8], uint64_t block, uint32_t out[16]) {
    uint32_t st[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u};
    for (int i = 0; i < 8; i++) st[4 + i] = key[i];
    st[12] = (uint32_t)block;
    st[13] = (uint32_t)(block >> 32);
    st[14] = 0;
    st[15] = 0;
    ref_chacha_core(st, 12, out);
}

uint32_t ref_rng_next_u32(ref_rng *r) {
    uint64_t block = r->pos >> 4;
    if (block != r->cached_block) {
        rng_block(r->key, block, r->buf);
        r->cached_block = block;
    }
    uint32_t w = r->buf[r->pos & 15];
    r->pos++;
    return w;
}

/* rand 0.8 Standard for f32: 24 high bits times 2^-24. */
float ref_rng_next_f32(ref_rng *r) {
    uint32_t v = ref_rng_next_u32(r) >> 8;
    return (float)v * (1.0f / 16777216.0f);
}

float ref_rng_word_f32(uint64_t seed, uint64_t word_index) {
    ref_rng r;
    ref_rng_seed_u64(&r, seed);
    ref_rng_set_pos(&r, word_index);
    return ref_rng_next_f32(&r);
}

/* ======================================================================== */
/* Sampler (inference/src/sampler.rs)                                       */
/* ======================================================================== */

/* f32::total_cmp key (core::f32::total_cmp). */
static inline int32_t total_key(float f) {
    int32_t i;
    memcpy(&i, &f, 4);
    i ^= (int32_t)(((uint32_t)(i >> 31)) >> 1);
    return i;
}

/* sampler.rs:91-97 */
int ref_is_deterministic(const ref_sampler *s) {
    return s->greedy || s->temperature <= FLT_EPSILON;
}

/* sampler.rs:217-224: max_by(total_cmp) keeps the LAST maximal index. */
int64_t ref_argmax(const float *v, int64_t n) {
    if (n <= 0) return 0;
    int64_t best = 0;
    int32_t bk = total_key(v[0]);
    for (int64_t i = 1; i < n; i++) {
        int32_t k = total_key(v[i]);
        if (k >= bk) {
            bk = k;
            best = i;
        }
    }
    return best;
}

/* sampler.rs:301-312 */
static int renormalize(float *p, int64_t n) {
    float sum = 0.0f;
    for (int64_t i = 0; i < n; i++) sum += p[i];
    if (!isfinite(sum) || sum <= 0.0f) return REF_ERR_CONFIG;
    for (int64_t i = 0; i < n; i++) p[i] /= sum;
    return REF_OK;
}

/* sampler.rs:280-299 with temperature 1.0 (filtered_probs divides first). */
static int softmax_t(const float *x, int64_t n, float temperature, float *out) {
    int found = 0;
    float mx = 0.0f;
    int32_t mk = 0;
    for (int64_t i = 0; i < n; i++) {
        if (isfinite(x[i])) {
            int32_t k = total_key(x[i]);
            if (!found || k >= mk) {
                mk = k;
                mx = x[i];
                found = 1;
            }
        }
    }
    if (!found) return REF_ERR_CONFIG;
    for (int64_t i = 0; i < n; i++)
        out[i] = isfinite(x[i]) ? expf((x[i] / temperature) - mx / temperature) : 0.0f;
    return renormalize(out, n);
}

typedef struct {
    float v;
    int64_t i;
} ranked_t;

/* Stable descending sort by total_cmp (slice::sort_by is stable). */
static int cmp_ranked_desc(const void *a, const void *b) {
    const ranked_t *x = (const ranked_t *)a, *y = (const ranked_t *)b;
    int32_t kx = total_key(x->v), ky = total_key(y->v);
    if (kx != ky) return kx > ky ? -1 : 1;
    return x->i < y->i ? -1 : (x->i > y->i);
}

/* Decision margins of the last filtered_probs call on this thread (test diagnostics:
   how far a rounding difference would have to move a value to change the kept set):
   the top-p cumulative sum's distance to top_p at its crossing, and the logit gap
   between the k-th and (k+1)-th ranked logits.  INFINITY when the filter is off. */
static __thread float g_topp_margin = INFINITY;
static __thread float g_topk_gap = INFINITY;
float ref_last_topp_margin(void) { return g_topp_margin; }
float ref_last_topk_gap(void) { return g_topk_gap; }

/* sampler.rs:226-278 */
static int filtered_probs(const float *logits, int64_t n, float temperature, int top_k,
                          float top_p, float *out) {
    g_topp_margin = INFINITY;
    g_topk_gap = INFINITY;
    float *masked = (float *)malloc(sizeof(float) * (size_t)n);
    unsigned char *allowed = (unsigned char *)malloc((size_t)n);
    if (!masked || !allowed) {
        free(masked);
        free(allowed);
        return REF_ERR_CONFIG;
    }
    memset(allowed, 1, (size_t)n);
    if (top_k > 0 && top_k < n) {
        ranked_t *r = (ranked_t *)malloc(sizeof(ranked_t) * (size_t)n);
        for (int64_t i = 0; i < n; i++) r[i] = (ranked_t){logits[i], i};
        qsort(r, (size_t)n, sizeof(ranked_t), cmp_ranked_desc);
        for (int64_t j = top_k; j < n; j++) allowed[r[j].i] = 0;
        g_topk_gap = fabsf(r[top_k - 1].v - r[top_k].v);
        if (!(g_topk_gap == g_topk_gap)) g_topk_gap = 0.0f;
        free(r);
    }
    for (int64_t i = 0; i < n; i++) masked[i] = allowed[i] ? logits[i] / temperature : -INFINITY;
    int st = softmax_t(masked, n, 1.0f, out);
    if (st == REF_OK && top_p > 0.0f && top_p < 1.0f) {
        ranked_t *r = (ranked_t *)malloc(sizeof(ranked_t) * (size_t)n);
        unsigned char *keep = (unsigned char *)calloc((size_t)n, 1);
        for (int64_t i = 0; i < n; i++) r[i] = (ranked_t){out[i], i};
        qsort(r, (size_t)n, sizeof(ranked_t), cmp_ranked_desc);
        float cum = 0.0f;
        for (int64_t j = 0; j < n; j++) {
            keep[r[j].i] = 1;
            float prev = cum;
            cum += r[j].v;
            if (cum >= top_p) {
                float a = cum - top_p, b = top_p - prev;
                g_topp_margin = a < b ? a : b;
                break;
            }
        }
        for (int64_t i = 0; i < n; i++)
            if (!keep[i]) out[i] = 0.0f;
        st = renormalize(out, n);
        free(r);
        free(keep);
    }
    free(masked);
    free(allowed);
    return st;
}

/* sampler.rs:102-118 (+ one_hot_argmax :211-215) */
int ref_probabilities(const ref_sampler *s, const float *logits, int64_t n, float *out) {
    g_topp_margin = INFINITY;
    g_topk_gap = INFINITY;
    if (n <= 0) return REF_ERR_SHAPE;
    if (s->greedy || !(s->temperature > FLT_EPSILON)) {
        memset(out, 0, sizeof(float) * (size_t)n);
        out[ref_argmax(logits, n)] = 1.0f;
        return REF_OK;
    }
    return filtered_probs(logits, n, s->temperature, s->top_k, s->top_p, out);
}

/* sampler.rs:314-335 */
int ref_validate_probabilities(const float *p, int64_t n) {
    if (n <= 0) return REF_ERR_SHAPE;
    for (int64_t i = 0; i < n; i++)
        if (!isfinite(p[i]) || p[i] < 0.0f) return REF_ERR_CONFIG;
    float sum = 0.0f;
    for (int64_t i = 0; i < n; i++) sum += p[i];
    if (!isfinite(sum) || fabsf(sum - 1.0f) > 1e-4f) return REF_ERR_CONFIG;
    return REF_OK;
}

/* sampler.rs:142-152 and sample_from_probs :337-347 (inverse CDF, draw <= cum). */
int ref_sample_probabilities(const ref_sampler *s, ref_rng *rng, const float *p, int64_t n,
                             uint32_t *out_token, float *out_draw, float *out_cdf_margin) {
    int st = ref_validate_probabilities(p, n);
    if (st) return st;
    if (out_cdf_margin) *out_cdf_margin = INFINITY;
    if (ref_is_deterministic(s)) {
        *out_token = (uint32_t)ref_argmax(p, n);
        if (out_draw) *out_draw = -1.0f;
        return REF_OK;
    }
    float draw = ref_rng_next_f32(rng);
    if (out_draw) *out_draw = draw;
    float cum = 0.0f, prev = 0.0f;
    for (int64_t i = 0; i < n; i++) {
        prev = cum;
        cum += p[i];
        if (draw <= cum) {
            *out_token = (uint32_t)i;
            if (out_cdf_margin) {
                float a = fabsf(cum - draw), b = fabsf(draw - prev);
                *out_cdf_margin = a < b ? a : b;
            }
            return REF_OK;
        }
    }
    *out_token = (uint32_t)(n - 1);
    if (out_cdf_margin) *out_cdf_margin = fabsf(draw - cum);
    return REF_OK;
}

/* speculative.rs:755-768 */
int ref_accept_proposal(const ref_sampler *s, ref_rng *rng, uint32_t token, const float *draft,
                        const float *target, int64_t n, int *accepted, float *out_ratio,
                        float *out_draw, int *drew) {
    *drew = 0;
    if (out_ratio) *out_ratio = NAN;
    if (out_draw) *out_draw = -1.0f;
    if (ref_is_deterministic(s)) {
        *accepted = ref_argmax(draft, n) == ref_argmax(target, n);
        return REF_OK;
    }
    float q = (int64_t)token < n ? draft[token] : 0.0f;
    float p = (int64_t)token < n ? target[token] : 0.0f;
    if (!(q > 0.0f)) {
        *accepted = 0;
        return REF_OK;
    }
    float u = ref_rng_next_f32(rng);
    *drew = 1;
    float ratio = p / q;
    float clipped = ratio < 1.0f ? ratio : 1.0f; /* f32::min(1.0) */
    if (isnan(ratio)) clipped = 1.0f;
    *accepted = u < clipped;
    if (out_ratio) *out_ratio = clipped;
    if (out_draw) *out_draw = u;
    return REF_OK;
}

/* speculative.rs:770-793 */
int ref_residual(const float *target, const float *draft, int64_t n, float *out) {
    for (int64_t i = 0; i < n; i++) {
        float d = target[i] - draft[i];
        out[i] = d > 0.0f ? d : 0.0f; /* f32::max(0.0): NaN -> 0.0 */
    }
    float sum = 0.0f;
    for (int64_t i = 0; i < n; i++) sum += out[i];
    if (!isfinite(sum) || sum <= FLT_EPSILON) return REF_ERR_CONFIG;
    for (int64_t i = 0; i < n; i++) out[i] /= sum;
    return REF_OK;
}

/*
 * One acceptance round per sequence, as the external-draft engine runs it
 * (speculative.rs:343-501): sequential accept_proposal over the proposals,
 * residual resample on the first rejection, optional bonus sample from the
 * row after the last proposal when everything is accepted.  The MTP engine
 * (mtp_speculative.rs:228-315) is the same with bonus = 0.
 */
int ref_accept_batch(int B, int K, int64_t V, const float *target, int target_rows,
                     const float *draft, const uint32_t *draft_tokens, const int32_t *n_proposals,
                     int bonus, const ref_sampler *s, const uint64_t *seeds,
                     const uint64_t *word_offsets, const float *uniforms,
                     ref_accept_result *out) {
    if (B <= 0 || K < 0 || V <= 0 || target_rows < K + (bonus ? 1 : 0)) return REF_ERR_SHAPE;
    float *p = (float *)malloc(sizeof(float) * (size_t)V);
    float *q = (float *)malloc(sizeof(float) * (size_t)V);
    float *r = (float *)malloc(sizeof(float) * (size_t)V);
    int status = REF_OK;
    for (int b = 0; b < B && status == REF_OK; b++) {
        ref_rng rng;
        ref_rng_seed_u64(&rng, seeds ? seeds[b] : 0);
        ref_rng_set_pos(&rng, word_offsets ? word_offsets[b] : 0);
        /* Explicit uniforms replace the keystream: a tiny shim RNG reading them in order. */
        int draw_idx = 0;
        ref_accept_result res = {0, -1, 0, 0, INFINITY, INFINITY};
        int np = n_proposals ? n_proposals[b] : K;
        if (np < 0 || np > K) {
            status = REF_ERR_SHAPE;
            break;
        }
        int rejected = 0;
        for (int i = 0; i < np; i++) {
            const float *tl = target + ((int64_t)b * target_rows + i) * V;
            const float *dl = draft + ((int64_t)b * K + i) * V;
            if ((status = ref_probabilities(s, tl, V, p))) break;
            if (g_topp_margin < 1e-6f) res.flags |= REF_FLAG_TOPP_NEAR;
            if ((status = ref_probabilities(s, dl, V, q))) break;
            if (g_topp_margin < 1e-6f) res.flags |= REF_FLAG_TOPP_NEAR;
            uint32_t tok = draft_tokens[(int64_t)b * K + i];
            int acc = 0, drew = 0;
            float ratio = 0, u = 0;
            if (uniforms && !ref_is_deterministic(s)) {
                float qq = (int64_t)tok < V ? q[tok] : 0.0f;
                float pp = (int64_t)tok < V ? p[tok] : 0.0f;
                if (qq > 0.0f) {
                    u = uniforms[(int64_t)b * (K + 1) + draw_idx];
                    drew = 1;
                    float rt = pp / qq;
                    ratio = rt < 1.0f ? rt : 1.0f;
                    acc = u < ratio;
                }
            } else {
                ref_accept_proposal(s, &rng, tok, q, p, V, &acc, &ratio, &u, &drew);
            }
            if (drew) {
                draw_idx++;
                float mg = fabsf(ratio - u);
                if (mg < res.ratio_margin) res.ratio_margin = mg;
                if (mg < 1e-5f) res.flags |= REF_FLAG_RATIO_NEAR;
            }
            if (acc) {
                res.accept_len++;
                continue;
            }
            rejected = 1;
            uint32_t tokr = 0;
            float cm = INFINITY;
            if (ref_is_deterministic(s)) {
                tokr = (uint32_t)ref_argmax(p, V);
            } else {
                if ((status = ref_residual(p, q, V, r))) break;
                if (uniforms) {
                    if ((status = ref_validate_probabilities(r, V))) break;
                    float draw = uniforms[(int64_t)b * (K + 1) + draw_idx];
                    float cum = 0.0f, prev = 0.0f;
                    tokr = (uint32_t)(V - 1);
                    for (int64_t j = 0; j < V; j++) {
                        prev = cum;
                        cum += r[j];
                        if (draw <= cum) {
                            tokr = (uint32_t)j;
                            break;
                        }
                    }
                    float a = fabsf(cum - draw), c = fabsf(draw - prev);
                    cm = a < c ? a : c;
                } else {
                    if ((status = ref_sample_probabilities(s, &rng, r, V, &tokr, NULL, &cm))) break;
                }
                draw_idx++;
            }
            res.token = (int32_t)tokr;
            res.cdf_margin = cm;
            break;
        }
        if (status) break;
        if (!rejected && bonus) {
            const float *tl = target + ((int64_t)b * target_rows + np) * V;
            if ((status = ref_probabilities(s, tl, V, p))) break;
            if (g_topp_margin < 1e-6f) res.flags |= REF_FLAG_TOPP_NEAR;
            uint32_t tokb = 0;
            float cm = INFINITY;
            if (uniforms && !ref_is_deterministic(s)) {
                if ((status = ref_validate_probabilities(p, V))) break;
                float draw = uniforms[(int64_t)b * (K + 1) + draw_idx];
                float cum = 0.0f, prev = 0.0f;
                tokb = (uint32_t)(V - 1);
                for (int64_t j = 0; j < V; j++) {
                    prev = cum;
                    cum += p[j];
                    if (draw <= cum) {
                        tokb = (uint32_t)j;
                        break;
                    }
                }
                float a = fabsf(cum - draw), c = fabsf(draw - prev);
                cm = a < c ? a : c;
            } else {
                if ((status = ref_sample_probabilities(s, &rng, p, V, &tokb, NULL, &cm))) break;
            }
            if (!ref_is_deterministic(s)) draw_idx++;
            res.token = (int32_t)tokb;
            res.cdf_margin = cm;
        }
        if (res.cdf_margin < 1e-6f) res.flags |= REF_FLAG_CDF_NEAR;
        res.draws = draw_idx;
        out[b] = res;
    }
    free(p);
    free(q);
    free(r);
    return status;
}

/* ======================================================================== */
/* Numeric formats                                                          */
/* ======================================================================== */

uint16_t ref_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t mant = x & 0x7FFFFFu;
    if (exp == 0xFFu) return (uint16_t)(sign | 0x7C00u | (mant ? (0x200u | (mant >> 13)) : 0));
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        mant |= 0x800000u;
        int shift = 14 - e;
        uint32_t half = 1u << (shift - 1);
        uint32_t rem = mant & ((1u << shift) - 1);
        uint32_t res = mant >> shift;
        if (rem > half || (rem == half && (res & 1u))) res++;
        return (uint16_t)(sign | res);
    }
    uint32_t res = ((uint32_t)e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (res & 1u))) res++;
    return (uint16_t)(sign | res);
}

float ref_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t mant = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            int e = -1;
            do {
                e++;
                mant <<= 1;
            } while ((mant & 0x400u) == 0);
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((mant & 0x3FFu) << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (mant << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t ref_f32_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7FFFu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

float ref_bf16_to_f32(uint16_t h) {
    uint32_t x = (uint32_t)h << 16;
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* ======================================================================== */
/* Quantisation (quant/src/int4.rs:7-91, absmax.rs:7-24, qat.rs:140-169)     */
/* ======================================================================== */

/* Rust f32::round: half away from zero. */
static inline float rust_roundf(float x) { return roundf(x); }

static inline float clampf(float v, float lo, float hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}

/* int4.rs:7-41 group statistics and codes for one group. */
static void i4_group(const float *g, int64_t len, unsigned char *codes, float *scale, float *zero) {
    float mn = INFINITY, mx = -INFINITY;
    for (int64_t i = 0; i < len; i++) {
        mn = fminf(mn, g[i]);
        mx = fmaxf(mx, g[i]);
    }
    float sc = fabsf(mx - mn) <= FLT_EPSILON ? 1.0f : (mx - mn) / 15.0f;
    float z = rust_roundf(-mn / sc);
    for (int64_t i = 0; i < len; i++)
        codes[i] = (unsigned char)clampf(rust_roundf((g[i] / sc) + z), 0.0f, 15.0f);
    *scale = sc;
    *zero = z;
}

/* int4.rs:45-53: low nibble holds the even index. */
static void pack_nibbles(const unsigned char *codes, int64_t n, uint8_t *packed) {
    for (int64_t i = 0; i < n; i += 2) {
        uint8_t lo = codes[i] & 0x0F;
        uint8_t hi = (i + 1 < n) ? (codes[i + 1] & 0x0F) : 0;
        packed[i / 2] = (uint8_t)(lo | (hi << 4));
    }
}

int ref_quantise_i4(const float *w, int64_t n, int64_t group, uint8_t *packed, float *scales,
                    float *zeros) {
    if (group <= 0) return REF_ERR_CONFIG;
    unsigned char *codes = (unsigned char *)malloc((size_t)n + 1);
    for (int64_t g0 = 0, gi = 0; g0 < n; g0 += group, gi++) {
        int64_t len = (n - g0) < group ? (n - g0) : group;
        i4_group(w + g0, len, codes + g0, &scales[gi], &zeros[gi]);
    }
    pack_nibbles(codes, n, packed);
    free(codes);
    return REF_OK;
}

/* int4.rs:70-91 */
int ref_dequantise_i4(const uint8_t *packed, int64_t n, int64_t group, const float *scales,
                      const float *zeros, float *out) {
    if (group <= 0) return REF_ERR_CONFIG;
    for (int64_t i = 0; i < n; i++) {
        uint8_t b = packed[i / 2];
        float qv = (float)((i & 1) ? (b >> 4) : (b & 0x0F));
        int64_t g = i / group;
        out[i] = (qv - zeros[g]) * scales[g];
    }
    return REF_OK;
}

/*
 * Build layout for GPTQ/AWQ-style INT4 g128: codes derived with the f32 group
 * scale exactly as int4.rs:7-41, scale and zero then stored as fp16 (the
 * "derive with f32, store f16" order of qat.rs:104-110).
 */
int ref_quantise_i4_f16(const float *w, int64_t n, int64_t group, uint8_t *packed,
                        uint16_t *scales_h, uint16_t *zeros_h) {
    if (group <= 0) return REF_ERR_CONFIG;
    int64_t ng = (n + group - 1) / group;
    float *sc = (float *)malloc(sizeof(float) * (size_t)ng);
    float *zz = (float *)malloc(sizeof(float) * (size_t)ng);
    ref_quantise_i4(w, n, group, packed, sc, zz);
    for (int64_t g = 0; g < ng; g++) {
        scales_h[g] = ref_f32_to_f16(sc[g]);
        zeros_h[g] = ref_f32_to_f16(zz[g]);
    }
    free(sc);
    free(zz);
    return REF_OK;
}

int ref_dequantise_i4_f16(const uint8_t *packed, int64_t n, int64_t group,
                          const uint16_t *scales_h, const uint16_t *zeros_h, float *out) {
    if (group <= 0) return REF_ERR_CONFIG;
    for (int64_t i = 0; i < n; i++) {
        uint8_t b = packed[i / 2];
        float qv = (float)((i & 1) ? (b >> 4) : (b & 0x0F));
        int64_t g = i / group;
        out[i] = (qv - ref_f16_to_f32(zeros_h[g])) * ref_f16_to_f32(scales_h[g]);
    }
    return REF_OK;
}

/*
 * Per-output-channel symmetric INT8 (qat.rs:155-169 fake_quant_symmetric with
 * ScaleAxes::OutputChannel and safe_scale): scale_r = max|W_r|/127, 1.0 when
 * the range is <= f32::EPSILON; q = clamp(round(W/scale_r), -127, 127).
 */
int ref_quantise_i8_rows(const float *w, int64_t rows, int64_t cols, int8_t *codes, float *scales) {
    for (int64_t r = 0; r < rows; r++) {
        const float *row = w + r * cols;
        float mx = 0.0f;
        for (int64_t c = 0; c < cols; c++) mx = fmaxf(mx, fabsf(row[c]));
        float sc = mx / 127.0f;
        if (mx <= FLT_EPSILON) sc = 1.0f;
        scales[r] = sc;
        for (int64_t c = 0; c < cols; c++)
            codes[r * cols + c] = (int8_t)clampf(rust_roundf(row[c] / sc), -127.0f, 127.0f);
    }
    return REF_OK;
}

/*
 * Build-defined INT8 KV cache row (one token, one kv-head): absmax rule of
 * absmax.rs:7-24 with the scale stored as fp16 after the codes are derived.
 * The reference's QuantisedKvCache (kv_quant.rs:16-56) re-quantises the whole
 * cache on every append and is not wired into inference; this per-token rule
 * is the semantic both the oracle and the GPU implement.
 */
int ref_quantise_kv_row(const float *x, int64_t n, int8_t *codes, uint16_t *scale_h) {
    float mx = 0.0f;
    for (int64_t i = 0; i < n; i++) mx = fmaxf(mx, fabsf(x[i]));
    float sc = mx <= FLT_EPSILON ? 1.0f : mx / 127.0f;
    for (int64_t i = 0; i < n; i++) codes[i] = (int8_t)clampf(rust_roundf(x[i] / sc), -127.0f, 127.0f);
    *scale_h = ref_f32_to_f16(sc);
    return REF_OK;
}

/* ======================================================================== */
/* Synthetic inputs (build-defined; the reference never seeds init, F12)    */
/* ======================================================================== */

uint64_t ref_splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

/* Box-Muller in f64 from a counter-based hash of (seed, stream, index). */
float ref_synth_normal(uint64_t seed, uint32_t stream, uint64_t index) {
    uint64_t base = ref_splitmix64(seed ^ ((uint64_t)stream * 0xD1B54A32D192ED03ull));
    uint64_t h = ref_splitmix64(base + index);
    double u1 = ((double)(h >> 40) + 1.0) * (1.0 / 16777216.0);
    double u2 = (double)((h >> 16) & 0xFFFFFFull) * (1.0 / 16777216.0);
    double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
    return (float)z;
}

void ref_synth_fill(uint64_t seed, uint32_t stream, int64_t n, float std, float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) out[i] = (float)((double)ref_synth_normal(seed, stream, (uint64_t)i) * (double)std);
}

void ref_synth_tokens(uint64_t seed, uint32_t stream, int64_t n, uint32_t vocab, uint32_t *out) {
    uint64_t base = ref_splitmix64(seed ^ ((uint64_t)stream * 0xD1B54A32D192ED03ull));
    for (int64_t i = 0; i < n; i++) out[i] = (uint32_t)(ref_splitmix64(base + (uint64_t)i) % vocab);
}

/* ======================================================================== */
/* Model (model/src/model.rs, nn/src/{block,attention,ffn,norm,rope,mtp}.rs) */
/* ======================================================================== */

enum { L_NORM1, L_WQ, L_WK, L_WV, L_WO, L_NORM2, L_WG, L_WU, L_WD, L_COUNT };
enum { H_TRUNK, H_TOKEN, H_NORM1, H_WQ, H_WK, H_WV, H_WO, H_NORM2, H_WG, H_WU, H_WD, H_OUT, H_COUNT };

typedef struct {
    char name[96];
    int64_t rows, cols;
    int32_t kind;
    float *data; /* effective (dequantised) f32 values */
} ref_tensor;

struct ref_model {
    ref_config cfg;
    int head_dim;
    int n_tensors;
    ref_tensor *t;
    float *rope_cos, *rope_sin; /* [max_seq_len, head_dim/2] */
};

struct ref_kv {
    const ref_model *m;
    int n_layers; /* copied so that freeing never touches the model */
    int capacity, len;
    float **k, **v; /* per layer [capacity, n_kv, head_dim], effective values */
};

static int tensor_id_embed(void) { return 0; }
static int tensor_id_layer(int l, int which) { return 1 + l * L_COUNT + which; }
static int tensor_id_final(const ref_config *c) { return 1 + c->n_layers * L_COUNT; }
static int tensor_id_head(const ref_config *c, int h, int which) {
    return 2 + c->n_layers * L_COUNT + h * H_COUNT + which;
}
/* Output projection of the model and of every MTP head (model.rs:239-262): the embedding,
   or lm_head.weight when the head is untied. */
static const float *lm_head_w(const ref_model *m) {
    return m->cfg.untied_lm_head ? m->t[m->n_tensors - 1].data : m->t[0].data;
}
static int n_heads_mtp(const ref_config *c) {
    return c->num_future_tokens > 1 ? c->num_future_tokens - 1 : 0;
}

static void set_info(ref_tensor *t, const char *name, int64_t rows, int64_t cols, int kind) {
    snprintf(t->name, sizeof(t->name), "%s", name);
    t->rows = rows;
    t->cols = cols;
    t->kind = kind;
}

/* RoPE inverse frequencies and cos / sin factor (inverse_frequencies_for_config,
   rope_scaling.rs:24-57): base (:6-11), linear (:46-52), NTK-aware theta (:14-22), YaRN
   (:60-92 with correction_range :107-130 and linear_ramp :132-139); validation and messages
   from RopeScalingConfig::validate (config.rs:52-96).  f64 arithmetic, results cast to f32.
   method: 0 none, 1 yarn, 2 ntk, 3 linear.  Returns 0, or -1 with the message in err. */
int ref_rope_frequencies(int hd, double theta, int max_seq_len, int method, double factor,
                         int original_max_seq_len, double beta_fast, double beta_slow,
                         double attn_factor, float *inv, float *attn, char *err, int err_cap) {
    int half = hd / 2;
#define ROPE_FAIL(...) do { if (err && err_cap > 0) snprintf(err, (size_t)err_cap, __VA_ARGS__); return -1; } while (0)
    if (hd <= 0 || hd % 2) ROPE_FAIL("RoPE head_dim must be non-zero and even");
    if (!(theta > 0.0) || !isfinite(theta)) ROPE_FAIL("RoPE theta must be finite and positive");
    *attn = 1.0f;
    for (int i = 0; i < half; i++) inv[i] = (float)(1.0 / pow(theta, 2.0 * (double)i / (double)hd));
    if (method == 0) return 0;
    if (!(factor > 1.0) || !isfinite(factor)) ROPE_FAIL("rope_scaling.factor must be finite and greater than 1.0");
    if (original_max_seq_len <= 0) ROPE_FAIL("rope_scaling.original_max_seq_len must be non-zero");
    if (max_seq_len < original_max_seq_len)
        ROPE_FAIL("max_seq_len %d must be >= rope_scaling.original_max_seq_len %d", max_seq_len, original_max_seq_len);
    if (hd <= 2) ROPE_FAIL("head_dim must be greater than 2 for RoPE scaling");
    if (!(attn_factor > 0.0) || !isfinite(attn_factor)) ROPE_FAIL("rope_scaling.attn_factor must be finite and positive");
    if (method == 1) {
        if (!(beta_fast > 0.0) || !(beta_slow > 0.0) || !isfinite(beta_fast) || !isfinite(beta_slow))
            ROPE_FAIL("rope_scaling beta values must be finite and positive");
        if (beta_fast <= beta_slow) ROPE_FAIL("rope_scaling.beta_fast must be greater than beta_slow");
    }
    *attn = (float)attn_factor;
    if (method == 3) {
        for (int i = 0; i < half; i++) inv[i] = inv[i] / (float)factor;
        return 0;
    }
    if (method == 2) {
        double th = theta * pow(factor, (double)hd / ((double)hd - 2.0));
        for (int i = 0; i < half; i++) inv[i] = (float)(1.0 / pow(th, 2.0 * (double)i / (double)hd));
        return 0;
    }
    if (method != 1) ROPE_FAIL("unknown rope_scaling method %d", method);
    {
        const double two_pi = 2.0 * 3.14159265358979323846, max_dim = half > 1 ? (double)(half - 1) : 0.0;
        double lo = floor((double)hd * log((double)original_max_seq_len / (beta_fast * two_pi)) / (2.0 * log(theta)));
        double hi = ceil((double)hd * log((double)original_max_seq_len / (beta_slow * two_pi)) / (2.0 * log(theta)));
        lo = lo < 0.0 ? 0.0 : (lo > max_dim ? max_dim : lo);
        hi = hi < 0.0 ? 0.0 : (hi > max_dim ? max_dim : hi);
        if (fabs(hi - lo) < 2.220446049250313e-16) hi += 0.001;
        for (int i = 0; i < half; i++) {
            double ex = 1.0 / pow(theta, 2.0 * (double)i / (double)hd), in = ex / factor;
            double ramp = ((double)i - lo) / (hi - lo);
            ramp = ramp < 0.0 ? 0.0 : (ramp > 1.0 ? 1.0 : ramp);
            inv[i] = (float)(in * ramp + ex * (1.0 - ramp));
        }
    }
    return 0;
#undef ROPE_FAIL
}

/* rope.rs:43-72: angle pos * freq in f32, cos and sin each times the attention factor. */
static void fill_rope(ref_model *m, const float *inv, float attn) {
    int half = m->head_dim / 2, S = m->cfg.max_seq_len;
    for (int p = 0; p < S; p++)
        for (int i = 0; i < half; i++) {
            float a = (float)p * inv[i];
            m->rope_cos[(size_t)p * half + i] = cosf(a) * attn;
            m->rope_sin[(size_t)p * half + i] = sinf(a) * attn;
        }
}

static void build_rope(ref_model *m) {
    int half = m->head_dim / 2, S = m->cfg.max_seq_len;
    m->rope_cos = (float *)malloc(sizeof(float) * (size_t)S * (size_t)half);
    m->rope_sin = (float *)malloc(sizeof(float) * (size_t)S * (size_t)half);
    float *inv = (float *)malloc(sizeof(float) * (size_t)half);
    float attn = 1.0f;
    ref_rope_frequencies(m->head_dim, (double)m->cfg.rope_theta, S, 0, 0, 0, 0, 0, 0, inv, &attn, NULL, 0);
    fill_rope(m, inv, attn);
    free(inv);
}

/* RopeCache::from_config (rope.rs:17-28) with cfg.rope_scaling set: rebuilds the tables. */
int ref_model_set_rope_scaling(ref_model *m, int method, double factor, int original_max_seq_len,
                               double beta_fast, double beta_slow, double attn_factor, char *err, int err_cap) {
    int half = m->head_dim / 2;
    float *inv = (float *)malloc(sizeof(float) * (size_t)(half > 0 ? half : 1)), attn = 1.0f;
    int r = ref_rope_frequencies(m->head_dim, (double)m->cfg.rope_theta, m->cfg.max_seq_len, method, factor,
                                 original_max_seq_len, beta_fast, beta_slow, attn_factor, inv, &attn, err, err_cap);
    if (!r) fill_rope(m, inv, attn);
    free(inv);
    return r;
}

ref_model *ref_model_create(const ref_config *cfg) {
    const ref_config *c = cfg;
    if (c->vocab_size <= 0 || c->hidden_dim <= 0 || c->ffn_dim <= 0 || c->n_layers <= 0 ||
        c->n_heads <= 0 || c->n_kv_heads <= 0 || c->max_seq_len <= 0)
        return NULL;
    if (c->hidden_dim % c->n_heads || c->n_heads % c->n_kv_heads) return NULL;
    if (c->untied_lm_head != 0 && c->untied_lm_head != 1) return NULL;
    /* model.rs:309-313 requires head_dim == 64; the benchmark shapes use 32 and 128,
       so that check is dropped here (documented divergence). */
    ref_model *m = (ref_model *)calloc(1, sizeof(ref_model));
    m->cfg = *c;
    m->head_dim = c->hidden_dim / c->n_heads;
    int nh = n_heads_mtp(c);
    m->n_tensors = 2 + c->n_layers * L_COUNT + nh * H_COUNT + c->untied_lm_head;
    m->t = (ref_tensor *)calloc((size_t)m->n_tensors, sizeof(ref_tensor));
    int64_t H = c->hidden_dim, F = c->ffn_dim, QD = (int64_t)c->n_heads * m->head_dim,
            KD = (int64_t)c->n_kv_heads * m->head_dim;
    char nm[96];
    set_info(&m->t[tensor_id_embed()], "embedding.weight", c->vocab_size, H, REF_T_EMBED);
    for (int l = 0; l < c->n_layers; l++) {
#define LT(which, suffix, r, cc, k)                                                                \
    snprintf(nm, sizeof(nm), "blocks.%d.%s", l, suffix);                                           \
    set_info(&m->t[tensor_id_layer(l, which)], nm, r, cc, k);
        LT(L_NORM1, "norm1.weight", 1, H, REF_T_NORM)
        LT(L_WQ, "attn.wq.weight", QD, H, REF_T_LINEAR)
        LT(L_WK, "attn.wk.weight", KD, H, REF_T_LINEAR)
        LT(L_WV, "attn.wv.weight", KD, H, REF_T_LINEAR)
        LT(L_WO, "attn.wo.weight", H, QD, REF_T_LINEAR)
        LT(L_NORM2, "norm2.weight", 1, H, REF_T_NORM)
        LT(L_WG, "ffn.w_gate.weight", F, H, REF_T_LINEAR)
        LT(L_WU, "ffn.w_up.weight", F, H, REF_T_LINEAR)
        LT(L_WD, "ffn.w_down.weight", H, F, REF_T_LINEAR)
#undef LT
    }
    set_info(&m->t[tensor_id_final(c)], "final_norm.weight", 1, H, REF_T_NORM);
    for (int h = 0; h < nh; h++) {
#define HT(which, suffix, r, cc, k)                                                                \
    snprintf(nm, sizeof(nm), "mtp.heads.%d.%s", h, suffix);                                        \
    set_info(&m->t[tensor_id_head(c, h, which)], nm, r, cc, k);
        HT(H_TRUNK, "trunk_norm.weight", 1, H, REF_T_NORM)
        HT(H_TOKEN, "token_norm.weight", 1, H, REF_T_NORM)
        HT(H_NORM1, "refine.norm1.weight", 1, H, REF_T_NORM)
        HT(H_WQ, "refine.attn.wq.weight", QD, H, REF_T_LINEAR)
        HT(H_WK, "refine.attn.wk.weight", KD, H, REF_T_LINEAR)
        HT(H_WV, "refine.attn.wv.weight", KD, H, REF_T_LINEAR)
        HT(H_WO, "refine.attn.wo.weight", H, QD, REF_T_LINEAR)
        HT(H_NORM2, "refine.norm2.weight", 1, H, REF_T_NORM)
        HT(H_WG, "refine.ffn.w_gate.weight", F, H, REF_T_LINEAR)
        HT(H_WU, "refine.ffn.w_up.weight", F, H, REF_T_LINEAR)
        HT(H_WD, "refine.ffn.w_down.weight", H, F, REF_T_LINEAR)
        HT(H_OUT, "output_norm.weight", 1, H, REF_T_NORM)
#undef HT
    }
    /* LmHead::untied_with_qat (model.rs:239-248), stored like the embedding */
    if (c->untied_lm_head) set_info(&m->t[m->n_tensors - 1], "lm_head.weight", c->vocab_size, H, REF_T_EMBED);
    for (int i = 0; i < m->n_tensors; i++) {
        size_t n = (size_t)(m->t[i].rows * m->t[i].cols);
        m->t[i].data = (float *)calloc(n, sizeof(float));
        if (!m->t[i].data) {
            ref_model_free(m);
            return NULL;
        }
        if (m->t[i].kind == REF_T_NORM)
            for (size_t j = 0; j < n; j++) m->t[i].data[j] = 1.0f; /* Init::Const(1.0), model.rs:110-121 */
    }
    build_rope(m);
    return m;
}

void ref_model_free(ref_model *m) {
    if (!m) return;
    for (int i = 0; i < m->n_tensors; i++) free(m->t[i].data);
    free(m->t);
    free(m->rope_cos);
    free(m->rope_sin);
    free(m);
}

int ref_model_num_tensors(const ref_model *m) { return m->n_tensors; }

int ref_model_tensor_info(const ref_model *m, int id, char *name, int name_cap, int64_t *rows,
                          int64_t *cols, int32_t *kind) {
    if (id < 0 || id >= m->n_tensors) return REF_ERR_SHAPE;
    if (name && name_cap > 0) snprintf(name, (size_t)name_cap, "%s", m->t[id].name);
    if (rows) *rows = m->t[id].rows;
    if (cols) *cols = m->t[id].cols;
    if (kind) *kind = m->t[id].kind;
    return REF_OK;
}

/* Store raw f32 values as the effective values the configured format yields. */
int ref_model_set_tensor(ref_model *m, int id, const float *raw) {
    if (id < 0 || id >= m->n_tensors) return REF_ERR_SHAPE;
    ref_tensor *t = &m->t[id];
    int64_t n = t->rows * t->cols;
    if (t->kind == REF_T_NORM) {
        memcpy(t->data, raw, sizeof(float) * (size_t)n);
        return REF_OK;
    }
    int fmt = t->kind == REF_T_EMBED ? (m->cfg.lm_head_format == 1 ? REF_W_BF16 : REF_W_F32)
                                     : m->cfg.weight_format;
    if (fmt == REF_W_F32) {
        memcpy(t->data, raw, sizeof(float) * (size_t)n);
    } else if (fmt == REF_W_BF16) {
        for (int64_t i = 0; i < n; i++) t->data[i] = ref_bf16_to_f32(ref_f32_to_bf16(raw[i]));
    } else if (fmt == REF_W_INT8_ROW) {
        int8_t *codes = (int8_t *)malloc((size_t)n);
        float *sc = (float *)malloc(sizeof(float) * (size_t)t->rows);
        ref_quantise_i8_rows(raw, t->rows, t->cols, codes, sc);
        for (int64_t r = 0; r < t->rows; r++)
            for (int64_t c = 0; c < t->cols; c++)
                t->data[r * t->cols + c] = (float)codes[r * t->cols + c] * sc[r];
        free(codes);
        free(sc);
    } else if (fmt == REF_W_INT4_G128) {
        if (t->cols % 128) return REF_ERR_SHAPE;
        int64_t ng = n / 128;
        uint8_t *packed = (uint8_t *)malloc((size_t)(n / 2));
        uint16_t *sh = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)ng);
        uint16_t *zh = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)ng);
        ref_quantise_i4_f16(raw, n, 128, packed, sh, zh);
        ref_dequantise_i4_f16(packed, n, 128, sh, zh, t->data);
        free(packed);
        free(sh);
        free(zh);
    } else {
        return REF_ERR_UNSUPPORTED;
    }
    return REF_OK;
}

int ref_model_get_tensor(const ref_model *m, int id, float *out) {
    if (id < 0 || id >= m->n_tensors) return REF_ERR_SHAPE;
    memcpy(out, m->t[id].data, sizeof(float) * (size_t)(m->t[id].rows * m->t[id].cols));
    return REF_OK;
}

/* Embedding and linears ~ N(0, std^2) (embedding.rs:12-19), norms 1.0. */
int ref_model_init_synthetic(ref_model *m, uint64_t seed, float std) {
    for (int i = 0; i < m->n_tensors; i++) {
        ref_tensor *t = &m->t[i];
        if (t->kind == REF_T_NORM) continue;
        int64_t n = t->rows * t->cols;
        float *raw = (float *)malloc(sizeof(float) * (size_t)n);
        if (!raw) return REF_ERR_CONFIG;
        ref_synth_fill(seed, (uint32_t)i, n, std, raw);
        int st = ref_model_set_tensor(m, i, raw);
        free(raw);
        if (st) return st;
    }
    return REF_OK;
}

/* ---------------- KV cache (nn/src/kvcache.rs:236-369, inference/src/kvcache.rs) ---------------- */

ref_kv *ref_kv_create(const ref_model *m, int capacity) {
    ref_kv *kv = (ref_kv *)calloc(1, sizeof(ref_kv));
    kv->m = m;
    kv->n_layers = m->cfg.n_layers;
    kv->capacity = capacity;
    int L = m->cfg.n_layers;
    size_t per = (size_t)capacity * (size_t)m->cfg.n_kv_heads * (size_t)m->head_dim;
    kv->k = (float **)calloc((size_t)L, sizeof(float *));
    kv->v = (float **)calloc((size_t)L, sizeof(float *));
    for (int l = 0; l < L; l++) {
        kv->k[l] = (float *)calloc(per, sizeof(float));
        kv->v[l] = (float *)calloc(per, sizeof(float));
        if (!kv->k[l] || !kv->v[l]) {
            ref_kv_free(kv);
            return NULL;
        }
    }
    return kv;
}

void ref_kv_free(ref_kv *kv) {
    if (!kv) return;
    for (int l = 0; l < kv->n_layers; l++) {
        if (kv->k) free(kv->k[l]);
        if (kv->v) free(kv->v[l]);
    }
    free(kv->k);
    free(kv->v);
    free(kv);
}

int ref_kv_len(const ref_kv *kv) { return kv->len; }

/* Rollback by index: restore() only rewinds len of shared storage (kvcache.rs:301-304,353-367). */
int ref_kv_truncate(ref_kv *kv, int new_len) {
    if (new_len < 0 || new_len > kv->len) return REF_ERR_SHAPE;
    kv->len = new_len;
    return REF_OK;
}

/* Store one token's K or V for one kv-head in the configured cache format. */
static void kv_store(const ref_model *m, float *dst, const float *src) {
    int hd = m->head_dim;
    if (m->cfg.kv_format == REF_KV_F32) {
        memcpy(dst, src, sizeof(float) * (size_t)hd);
    } else if (m->cfg.kv_format == REF_KV_F16) {
        for (int i = 0; i < hd; i++) dst[i] = ref_f16_to_f32(ref_f32_to_f16(src[i]));
    } else {
        int8_t codes[512];
        uint16_t sh;
        ref_quantise_kv_row(src, hd, codes, &sh);
        float sc = ref_f16_to_f32(sh);
        for (int i = 0; i < hd; i++) dst[i] = (float)codes[i] * sc;
    }
}

/* Synthetic cache contents (post-RoPE K and V ~ N(0,1)) for long-context benches. */
int ref_kv_fill_synthetic(ref_kv *kv, uint64_t seed, int len) {
    const ref_model *m = kv->m;
    if (len > kv->capacity) return REF_ERR_SHAPE;
    int hd = m->head_dim, nkv = m->cfg.n_kv_heads;
    float *tmp = (float *)malloc(sizeof(float) * (size_t)hd);
    for (int l = 0; l < m->cfg.n_layers; l++)
        for (int which = 0; which < 2; which++) {
            float *base = which ? kv->v[l] : kv->k[l];
            uint32_t stream = 0x4B560000u + (uint32_t)(l * 2 + which);
            for (int t = 0; t < len; t++)
                for (int h = 0; h < nkv; h++) {
                    uint64_t off = ((uint64_t)t * nkv + h) * hd;
                    for (int i = 0; i < hd; i++) tmp[i] = ref_synth_normal(seed, stream, off + i);
                    kv_store(m, base + off, tmp);
                }
        }
    free(tmp);
    kv->len = len;
    return REF_OK;
}

/* ---------------- layer math ---------------- */

static inline float dotf(const float *a, const float *b, int64_t n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int64_t k = 0;
    for (; k + 8 <= n; k += 8)
        for (int j = 0; j < 8; j++) acc[j] = fmaf(a[k + j], b[k + j], acc[j]);
    float s = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
    for (; k < n; k++) s = fmaf(a[k], b[k], s);
    return s;
}

/* QatLinear::forward (qat.rs:315-348): y[M,N] = x[M,K] . W[N,K]^T. */
static void linear(const float *x, int M, int64_t K, const float *W, int64_t N, float *y, int nt) {
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t n = 0; n < N; n++) {
        const float *w = W + n * K;
        for (int m = 0; m < M; m++) y[(int64_t)m * N + n] = dotf(x + (int64_t)m * K, w, K);
    }
}

/* cpu_rms_norm_scalar (kernel/src/cpu/simd_norm.rs:51-57). */
static void rms_norm(const float *x, int M, int64_t H, const float *w, float eps, float *y) {
    for (int m = 0; m < M; m++) {
        const float *r = x + (int64_t)m * H;
        float ss = 0.0f;
        for (int64_t i = 0; i < H; i++) ss += r[i] * r[i];
        float inv = 1.0f / sqrtf(ss / (float)H + eps);
        for (int64_t i = 0; i < H; i++) y[(int64_t)m * H + i] = r[i] * inv * w[i];
    }
}

/* RopeCache::apply_rotate (rope.rs:107-126): half-split rotation. */
static void rope_apply(const ref_model *m, float *x, int S, int n_heads, int pos0) {
    int hd = m->head_dim, half = hd / 2;
    for (int s = 0; s < S; s++) {
        const float *c = m->rope_cos + (size_t)(pos0 + s) * half;
        const float *sn = m->rope_sin + (size_t)(pos0 + s) * half;
        for (int h = 0; h < n_heads; h++) {
            float *v = x + ((int64_t)s * n_heads + h) * hd;
            for (int i = 0; i < half; i++) {
                float x1 = v[i], x2 = v[i + half];
                v[i] = x1 * c[i] - x2 * sn[i];
                v[i + half] = x1 * sn[i] + x2 * c[i];
            }
        }
    }
}

/*
 * Causal attention, one online-softmax pass per (head, query) row
 * (kernel/src/cpu/parallel_attn.rs:190-233); query head h reads kv head
 * h % n_kv (repeat_heads, attention.rs:415-428); causal shift kv_len - q_len.
 * k/v are laid out [kv_len, n_kv, head_dim].
 */
static void attention(const ref_model *m, const float *q, int S, const float *k, const float *v,
                      int kv_len, float *out, int nt) {
    int hd = m->head_dim, nh = m->cfg.n_heads, nkv = m->cfg.n_kv_heads;
    float scale = (float)(1.0 / sqrt((double)hd));
    int shift = kv_len - S;
    if (shift < 0) shift = 0;
#pragma omp parallel for num_threads(nt) schedule(static) collapse(2)
    for (int h = 0; h < nh; h++)
        for (int s = 0; s < S; s++) {
            const float *qr = q + ((int64_t)s * nh + h) * hd;
            float *o = out + ((int64_t)s * nh + h) * hd;
            int kh = h % nkv;
            for (int d = 0; d < hd; d++) o[d] = 0.0f;
            float run_max = -INFINITY, run_sum = 0.0f;
            for (int t = 0; t < kv_len; t++) {
                if (t > shift + s) continue;
                const float *kr = k + ((int64_t)t * nkv + kh) * hd;
                const float *vr = v + ((int64_t)t * nkv + kh) * hd;
                float dot = 0.0f;
                for (int d = 0; d < hd; d++) dot += qr[d] * kr[d];
                float score = dot * scale + 0.0f;
                float next_max = fmaxf(run_max, score);
                float old_scale = expf(run_max - next_max);
                float new_scale = expf(score - next_max);
                for (int d = 0; d < hd; d++) o[d] = o[d] * old_scale + new_scale * vr[d];
                run_sum = run_sum * old_scale + new_scale;
                run_max = next_max;
            }
            if (run_sum > 0.0f) {
                float inv = 1.0f / run_sum;
                for (int d = 0; d < hd; d++) o[d] *= inv;
            }
        }
}

typedef struct {
    const float *norm1, *wq, *wk, *wv, *wo, *norm2, *wg, *wu, *wd;
} block_w;

static block_w layer_weights(const ref_model *m, int l) {
    block_w b;
    b.norm1 = m->t[tensor_id_layer(l, L_NORM1)].data;
    b.wq = m->t[tensor_id_layer(l, L_WQ)].data;
    b.wk = m->t[tensor_id_layer(l, L_WK)].data;
    b.wv = m->t[tensor_id_layer(l, L_WV)].data;
    b.wo = m->t[tensor_id_layer(l, L_WO)].data;
    b.norm2 = m->t[tensor_id_layer(l, L_NORM2)].data;
    b.wg = m->t[tensor_id_layer(l, L_WG)].data;
    b.wu = m->t[tensor_id_layer(l, L_WU)].data;
    b.wd = m->t[tensor_id_layer(l, L_WD)].data;
    return b;
}

static block_w head_weights(const ref_model *m, int h) {
    const ref_config *c = &m->cfg;
    block_w b;
    b.norm1 = m->t[tensor_id_head(c, h, H_NORM1)].data;
    b.wq = m->t[tensor_id_head(c, h, H_WQ)].data;
    b.wk = m->t[tensor_id_head(c, h, H_WK)].data;
    b.wv = m->t[tensor_id_head(c, h, H_WV)].data;
    b.wo = m->t[tensor_id_head(c, h, H_WO)].data;
    b.norm2 = m->t[tensor_id_head(c, h, H_NORM2)].data;
    b.wg = m->t[tensor_id_head(c, h, H_WG)].data;
    b.wu = m->t[tensor_id_head(c, h, H_WU)].data;
    b.wd = m->t[tensor_id_head(c, h, H_WD)].data;
    return b;
}

/*
 * TransformerBlock::forward (block.rs:331-350) with GroupedQueryAttention::forward
 * (attention.rs:170-222) and SwiGluFfn::forward (ffn.rs:29-37).  With kv_k/kv_v
 * set, the new K/V rows are stored in the cache format at rows pos0.. and the
 * attention reads the cache; otherwise the local K/V are used as is.
 */
static void block_forward(const ref_model *m, const block_w *w, float *x, int S, int pos0,
                          float *kv_k, float *kv_v, int nt) {
    const ref_config *c = &m->cfg;
    int64_t H = c->hidden_dim, F = c->ffn_dim;
    int hd = m->head_dim, nh = c->n_heads, nkv = c->n_kv_heads;
    int64_t QD = (int64_t)nh * hd, KD = (int64_t)nkv * hd;
    float *xn = (float *)malloc(sizeof(float) * (size_t)(S * H));
    float *q = (float *)malloc(sizeof(float) * (size_t)(S * QD));
    float *k = (float *)malloc(sizeof(float) * (size_t)(S * KD));
    float *v = (float *)malloc(sizeof(float) * (size_t)(S * KD));
    float *o = (float *)malloc(sizeof(float) * (size_t)(S * QD));
    float *y = (float *)malloc(sizeof(float) * (size_t)(S * H));
    float *g = (float *)malloc(sizeof(float) * (size_t)(S * F));
    float *u = (float *)malloc(sizeof(float) * (size_t)(S * F));

    rms_norm(x, S, H, w->norm1, c->norm_eps, xn);
    linear(xn, S, H, w->wq, QD, q, nt);
    linear(xn, S, H, w->wk, KD, k, nt);
    linear(xn, S, H, w->wv, KD, v, nt);
    rope_apply(m, q, S, nh, pos0);
    rope_apply(m, k, S, nkv, pos0);
    if (kv_k) {
        for (int s = 0; s < S; s++)
            for (int h = 0; h < nkv; h++) {
                int64_t src = ((int64_t)s * nkv + h) * hd;
                int64_t dst = ((int64_t)(pos0 + s) * nkv + h) * hd;
                kv_store(m, kv_k + dst, k + src);
                kv_store(m, kv_v + dst, v + src);
            }
        attention(m, q, S, kv_k, kv_v, pos0 + S, o, nt);
    } else {
        attention(m, q, S, k, v, S, o, nt);
    }
    linear(o, S, QD, w->wo, H, y, nt);
    for (int64_t i = 0; i < S * H; i++) x[i] = x[i] + y[i];

    rms_norm(x, S, H, w->norm2, c->norm_eps, xn);
    linear(xn, S, H, w->wg, F, g, nt);
    linear(xn, S, H, w->wu, F, u, nt);
    for (int64_t i = 0; i < S * F; i++) {
        float gv = g[i];
        float silu = gv / (1.0f + expf(-gv)); /* candle silu: x / (1 + exp(-x)) */
        g[i] = silu * u[i];
    }
    linear(g, S, F, w->wd, H, y, nt);
    for (int64_t i = 0; i < S * H; i++) x[i] = x[i] + y[i];

    free(xn);
    free(q);
    free(k);
    free(v);
    free(o);
    free(y);
    free(g);
    free(u);
}

/*
 * AarambhModel::forward_with_cache_output (model.rs:529-587): embedding gather,
 * blocks, final RMSNorm, tied LM head.  offset must not exceed the cache length;
 * a smaller offset rewinds the cache first (rollback by index).
 */
int ref_forward_layers(const ref_model *m, ref_kv *kv, const uint32_t *ids, int S, int offset,
                       int n_layers, int with_head, float *logits, int nt) {
    const ref_config *c = &m->cfg;
    if (S <= 0) return REF_ERR_SHAPE;
    if (offset + S > c->max_seq_len) return REF_ERR_SHAPE; /* check_token_ids, model.rs:886-907 */
    if (!kv || offset > kv->len || offset + S > kv->capacity) return REF_ERR_SHAPE;
    int64_t H = c->hidden_dim, V = c->vocab_size;
    for (int s = 0; s < S; s++)
        if ((int64_t)ids[s] >= V) return REF_ERR_SHAPE;
    kv->len = offset;
    float *x = (float *)malloc(sizeof(float) * (size_t)(S * H));
    const float *emb = m->t[tensor_id_embed()].data;
    for (int s = 0; s < S; s++) memcpy(x + s * H, emb + (int64_t)ids[s] * H, sizeof(float) * (size_t)H);
    int L = n_layers < c->n_layers ? n_layers : c->n_layers;
    for (int l = 0; l < L; l++) {
        block_w w = layer_weights(m, l);
        block_forward(m, &w, x, S, offset, kv->k[l], kv->v[l], nt);
    }
    kv->len = offset + S;
    if (with_head) {
        float *hn = (float *)malloc(sizeof(float) * (size_t)(S * H));
        rms_norm(x, S, H, m->t[tensor_id_final(c)].data, c->norm_eps, hn);
        if (logits) linear(hn, S, H, lm_head_w(m), V, logits, nt);
        free(hn);
    }
    free(x);
    return REF_OK;
}

int ref_forward(const ref_model *m, ref_kv *kv, const uint32_t *ids, int S, int offset,
                float *logits, float *hidden, int nt) {
    const ref_config *c = &m->cfg;
    if (S <= 0) return REF_ERR_SHAPE;
    if (offset + S > c->max_seq_len) return REF_ERR_SHAPE;
    if (!kv || offset > kv->len || offset + S > kv->capacity) return REF_ERR_SHAPE;
    int64_t H = c->hidden_dim, V = c->vocab_size;
    for (int s = 0; s < S; s++)
        if ((int64_t)ids[s] >= V) return REF_ERR_SHAPE;
    kv->len = offset;
    float *x = (float *)malloc(sizeof(float) * (size_t)(S * H));
    const float *emb = m->t[tensor_id_embed()].data;
    for (int s = 0; s < S; s++) memcpy(x + s * H, emb + (int64_t)ids[s] * H, sizeof(float) * (size_t)H);
    for (int l = 0; l < c->n_layers; l++) {
        block_w w = layer_weights(m, l);
        block_forward(m, &w, x, S, offset, kv->k[l], kv->v[l], nt);
    }
    kv->len = offset + S;
    float *hn = (float *)malloc(sizeof(float) * (size_t)(S * H));
    rms_norm(x, S, H, m->t[tensor_id_final(c)].data, c->norm_eps, hn);
    if (hidden) memcpy(hidden, hn, sizeof(float) * (size_t)(S * H));
    if (logits) linear(hn, S, H, lm_head_w(m), V, logits, nt);
    free(hn);
    free(x);
    return REF_OK;
}

/*
 * AarambhModel::forward_mtp_head (model.rs:783-817) -> MtpHead::forward
 * (mtp.rs:104-114): local = [trunk_norm(anchor), token_norm(emb(ids))], one
 * refine block from position 0 without a cache, output_norm on the last row,
 * shared LM head.  head h has offset h+2 and needs h+1 intervening ids.
 */
int ref_mtp_head(const ref_model *m, int head, const float *anchor, const uint32_t *ids,
                 int n_ids, float *logits, int nt) {
    const ref_config *c = &m->cfg;
    if (head < 0 || head >= n_heads_mtp(c)) return REF_ERR_CONFIG;
    if (n_ids != head + 1) return REF_ERR_SHAPE;
    int64_t H = c->hidden_dim, V = c->vocab_size;
    int L = n_ids + 1;
    float *x = (float *)malloc(sizeof(float) * (size_t)(L * H));
    const float *emb = m->t[tensor_id_embed()].data;
    rms_norm(anchor, 1, H, m->t[tensor_id_head(c, head, H_TRUNK)].data, c->norm_eps, x);
    for (int i = 0; i < n_ids; i++) {
        if ((int64_t)ids[i] >= V) {
            free(x);
            return REF_ERR_SHAPE;
        }
        rms_norm(emb + (int64_t)ids[i] * H, 1, H, m->t[tensor_id_head(c, head, H_TOKEN)].data,
                 c->norm_eps, x + (int64_t)(i + 1) * H);
    }
    block_w w = head_weights(m, head);
    block_forward(m, &w, x, L, 0, NULL, NULL, nt);
    float *hn = (float *)malloc(sizeof(float) * (size_t)H);
    rms_norm(x + (int64_t)(L - 1) * H, 1, H, m->t[tensor_id_head(c, head, H_OUT)].data,
             c->norm_eps, hn);
    linear(hn, 1, H, lm_head_w(m), V, logits, nt);
    free(hn);
    free(x);
    return REF_OK;
}

/* ======================================================================== */
/* Engines                                                                  */
/* ======================================================================== */

#define EOS_ID 0u /* tokenizer/src/special.rs:33 */

/* top-two gap of a logits row (greedy near-tie measure) */
static float top2_gap(const float *v, int64_t n) {
    float a = -INFINITY, b = -INFINITY;
    for (int64_t i = 0; i < n; i++) {
        if (v[i] > a) {
            b = a;
            a = v[i];
        } else if (v[i] > b) {
            b = v[i];
        }
    }
    return a - b;
}

/* Sampler::top_candidates_from_probabilities (sampler.rs:188-208): stable descending
   sort of the distribution truncated to k (engine.rs:70: top_candidates = 5).  The
   engines below compute it for every committed token (mtp_speculative.rs:247-250,
   speculative.rs); when a sink is set (test harness, single-threaded) the k
   candidates of committed token `slot` are stored there. */
static uint32_t *g_cand_ids;
static float *g_cand_probs;
static int g_cand_cap;

void ref_set_candidate_sink(uint32_t *ids, float *probs, int cap) {
    g_cand_ids = ids;
    g_cand_probs = probs;
    g_cand_cap = ids && probs ? cap : 0;
}

/* Per-round trace of the engines (test harness, single-threaded): the state a round
   starts from (committed tokens, keystream position) and how close its decisions came
   to flipping, so a device run can be compared round by round and restarted from the
   oracle's state after a near-tie. */
static ref_round *g_round_buf;
static int g_round_cap;
static int *g_round_count;

void ref_set_round_sink(ref_round *buf, int cap, int *count) {
    g_round_buf = buf;
    g_round_cap = buf && count ? cap : 0;
    g_round_count = count;
    if (count) *count = 0;
}

static void round_margin_prob(ref_round *r, float m) {
    if (m < r->prob_margin) r->prob_margin = m;
}
static void round_margin_logit(ref_round *r, float m) {
    if (m < r->logit_gap) r->logit_gap = m;
}
/* margins of the distribution ref_probabilities just built */
static void round_margin_filter(ref_round *r) {
    round_margin_prob(r, g_topp_margin);
    round_margin_logit(r, g_topk_gap);
}
static void round_begin(ref_round *r, int committed, const ref_rng *rng) {
    memset(r, 0, sizeof(*r));
    r->rng_pos_before = rng->pos;
    r->committed_before = committed;
    r->prob_margin = INFINITY;
    r->logit_gap = INFINITY;
}
static void round_end(ref_round *r, int committed, const ref_rng *rng) {
    r->committed_after = committed;
    r->rng_pos_after = rng->pos;
    if (g_round_count && *g_round_count < g_round_cap) g_round_buf[*g_round_count] = *r;
    if (g_round_count) (*g_round_count)++;
}

void ref_top_candidates(const float *p, int64_t n, int k, uint32_t *ids, float *probs) {
    ranked_t *r = (ranked_t *)malloc(sizeof(ranked_t) * (size_t)n);
    for (int64_t i = 0; i < n; i++) r[i] = (ranked_t){p[i], i};
    qsort(r, (size_t)n, sizeof(ranked_t), cmp_ranked_desc);
    for (int i = 0; i < k; i++) {
        ids[i] = i < n ? (uint32_t)r[i].i : UINT32_MAX;
        probs[i] = i < n ? r[i].v : 0.0f;
    }
    free(r);
}

static void top_candidates(const float *p, int64_t n, int k, int slot) {
    uint32_t ids[16];
    float probs[16];
    ref_top_candidates(p, n, k, ids, probs);
    if (slot >= 0 && slot < g_cand_cap)
        for (int i = 0; i < k; i++) {
            g_cand_ids[(int64_t)slot * k + i] = ids[i];
            g_cand_probs[(int64_t)slot * k + i] = probs[i];
        }
}

/*
 * MtpSpeculativeEngine::generate_with_callback (mtp_speculative.rs:86-336),
 * with the thinking/tool controllers inactive (ThinkingMode::None, no tools).
 */
int ref_mtp_generate(const ref_model *m, const uint32_t *prompt, int prompt_len,
                     int max_new_tokens, int num_draft_tokens, const ref_sampler *s,
                     uint64_t seed, int nt, uint32_t *out_tokens, int *out_len,
                     int *finish_reason, ref_spec_stats *stats, float *out_min_gap) {
    const ref_config *c = &m->cfg;
    int nheads = n_heads_mtp(c);
    if (nheads == 0) return REF_ERR_CONFIG;
    if (num_draft_tokens < 2 || num_draft_tokens > c->num_future_tokens) return REF_ERR_CONFIG;
    if (prompt_len <= 0) return REF_ERR_SHAPE;
    if (prompt_len >= c->max_seq_len) return REF_ERR_SHAPE;
    int available = c->max_seq_len - prompt_len;
    int max_new = max_new_tokens < available ? max_new_tokens : available;
    memset(stats, 0, sizeof(*stats));
    *out_len = 0;
    *finish_reason = REF_FINISH_MAX_TOKENS;
    float min_gap = INFINITY;
    if (max_new == 0) {
        *finish_reason = REF_FINISH_CONTEXT_LIMIT;
        if (out_min_gap) *out_min_gap = min_gap;
        return REF_OK;
    }
    int64_t V = c->vocab_size, H = c->hidden_dim;
    int K = num_draft_tokens;
    ref_rng rng;
    ref_rng_seed_u64(&rng, seed);
    ref_kv *kv = ref_kv_create(m, c->max_seq_len);
    if (!kv) return REF_ERR_CONFIG;
    float *plog = (float *)malloc(sizeof(float) * (size_t)(prompt_len * V));
    float *phid = (float *)malloc(sizeof(float) * (size_t)(prompt_len * H));
    int st = ref_forward(m, kv, prompt, prompt_len, 0, plog, phid, nt);
    float *target_next = (float *)malloc(sizeof(float) * (size_t)V);
    float *anchor = (float *)malloc(sizeof(float) * (size_t)H);
    memcpy(target_next, plog + (int64_t)(prompt_len - 1) * V, sizeof(float) * (size_t)V);
    memcpy(anchor, phid + (int64_t)(prompt_len - 1) * H, sizeof(float) * (size_t)H);
    free(plog);
    free(phid);

    float *dist = (float *)malloc(sizeof(float) * (size_t)(K * V)); /* proposal distributions */
    float *mlog = (float *)malloc(sizeof(float) * (size_t)V);
    float *vlog = (float *)malloc(sizeof(float) * (size_t)(K * V));
    float *vhid = (float *)malloc(sizeof(float) * (size_t)(K * H));
    float *pt = (float *)malloc(sizeof(float) * (size_t)V);
    float *res = (float *)malloc(sizeof(float) * (size_t)V);
    uint32_t *props = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)K);
    uint32_t *replay = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)(K + 1));
    int n_out = 0;

    while (st == REF_OK && n_out < max_new) {
        int remaining = max_new - n_out;
        int count = K < remaining ? K : remaining;
        int base = kv->len;
        int np = 0;
        ref_round rr;
        round_begin(&rr, n_out, &rng);
        for (int pi = 0; pi < count; pi++) {
            const float *lg;
            if (pi == 0) {
                lg = target_next;
            } else {
                if ((st = ref_mtp_head(m, pi - 1, anchor, props, pi, mlog, nt))) break;
                stats->mtp_head_forwards++;
                lg = mlog;
            }
            if (ref_is_deterministic(s)) {
                float gp = top2_gap(lg, V);
                if (gp < min_gap) min_gap = gp;
                round_margin_logit(&rr, gp);
            }
            if ((st = ref_probabilities(s, lg, V, dist + (int64_t)pi * V))) break;
            round_margin_filter(&rr);
            uint32_t tok;
            float cmp = INFINITY;
            if ((st = ref_sample_probabilities(s, &rng, dist + (int64_t)pi * V, V, &tok, NULL, &cmp)))
                break;
            if (!ref_is_deterministic(s)) round_margin_prob(&rr, cmp);
            props[np++] = tok;
            stats->draft_tokens_proposed++;
            if (tok == EOS_ID) break;
        }
        if (st) break;
        if ((st = ref_forward(m, kv, props, np, base, vlog, vhid, nt))) break;
        stats->rounds++;
        stats->target_decode_forwards++;
        int rejected = 0, done = 0;
        rr.proposed = np;
        for (int i = 0; i < np; i++) {
            const float *tl = i == 0 ? target_next : vlog + (int64_t)(i - 1) * V;
            if (ref_is_deterministic(s)) {
                float gp = top2_gap(tl, V);
                if (gp < min_gap) min_gap = gp;
                round_margin_logit(&rr, gp);
            }
            if ((st = ref_probabilities(s, tl, V, pt))) break;
            round_margin_filter(&rr);
            int acc = 0, drew = 0;
            float ratio = 0.0f, u = 0.0f;
            ref_accept_proposal(s, &rng, props[i], dist + (int64_t)i * V, pt, V, &acc, &ratio, &u, &drew);
            if (drew) round_margin_prob(&rr, fabsf(ratio - u));
            top_candidates(pt, V, 5, n_out);
            if (acc) {
                rr.accepted++;
                stats->draft_tokens_accepted++;
                if (props[i] == EOS_ID) {
                    *finish_reason = REF_FINISH_EOS;
                    done = 1;
                    break;
                }
                out_tokens[n_out++] = props[i];
                if (n_out == max_new) {
                    done = 1;
                    break;
                }
                continue;
            }
            rejected = 1;
            uint32_t repl;
            if (ref_is_deterministic(s)) {
                if ((st = ref_sample_probabilities(s, &rng, pt, V, &repl, NULL, NULL))) break;
            } else {
                float cmr = INFINITY;
                if ((st = ref_residual(pt, dist + (int64_t)i * V, V, res))) break;
                if ((st = ref_sample_probabilities(s, &rng, res, V, &repl, NULL, &cmr))) break;
                round_margin_prob(&rr, cmr);
            }
            kv->len = base; /* target_cache.restore(snapshot) */
            if (repl == EOS_ID) {
                *finish_reason = REF_FINISH_EOS;
                done = 1;
                break;
            }
            out_tokens[n_out++] = repl;
            for (int j = 0; j < i; j++) replay[j] = props[j];
            replay[i] = repl;
            if ((st = ref_forward(m, kv, replay, i + 1, base, vlog, vhid, nt))) break;
            stats->target_decode_forwards++;
            memcpy(target_next, vlog + (int64_t)i * V, sizeof(float) * (size_t)V);
            memcpy(anchor, vhid + (int64_t)i * H, sizeof(float) * (size_t)H);
            break;
        }
        if (!st) round_end(&rr, n_out, &rng);
        if (st || done) break;
        if (rejected) continue;
        memcpy(target_next, vlog + (int64_t)(np - 1) * V, sizeof(float) * (size_t)V);
        memcpy(anchor, vhid + (int64_t)(np - 1) * H, sizeof(float) * (size_t)H);
    }
    if (st == REF_OK) {
        if (n_out == available && *finish_reason == REF_FINISH_MAX_TOKENS)
            *finish_reason = REF_FINISH_CONTEXT_LIMIT;
        stats->draft_tokens_rejected = stats->draft_tokens_proposed - stats->draft_tokens_accepted;
        if (stats->draft_tokens_rejected < 0) stats->draft_tokens_rejected = 0;
    }
    *out_len = n_out;
    if (out_min_gap) *out_min_gap = min_gap;
    free(dist);
    free(mlog);
    free(vlog);
    free(vhid);
    free(pt);
    free(res);
    free(props);
    free(replay);
    free(target_next);
    free(anchor);
    ref_kv_free(kv);
    return st;
}

/*
 * SpeculativeEngine::generate_with_callback (speculative.rs:175-516): external
 * draft model, controllers inactive (ThinkingMode::None, no tools).  Per round
 * (speculative.rs:251-509): the draft proposes up to k tokens autoregressively
 * (one sampling draw each, stopping after an EOS proposal), the target verifies
 * [pending?] + proposals in one forward, proposals are tested in order; on the
 * first rejection both caches are restored, the target replays
 * [pending?] + accepted proposals, the draft replays the accepted proposals and
 * then the replacement, which becomes the pending target token; when every
 * proposal is accepted a bonus token is sampled from the row after the last
 * proposal, fed to the draft and kept pending.  The shared context limit is
 * min(target, draft) max_seq_len (speculative.rs:203-212).
 */
int ref_spec_generate(const ref_model *tm, const ref_model *dm, const uint32_t *prompt, int prompt_len,
                      int max_new_tokens, int num_draft_tokens, const ref_sampler *s, uint64_t seed,
                      int nt, uint32_t *out_tokens, int *out_len, int *finish_reason,
                      ref_spec_stats *stats, float *out_min_gap) {
    const ref_config *tc = &tm->cfg, *dc = &dm->cfg;
    if (num_draft_tokens <= 0) return REF_ERR_CONFIG; /* speculative.rs:104-108 */
    if (tc->vocab_size != dc->vocab_size) return REF_ERR_CONFIG;
    if (prompt_len <= 0) return REF_ERR_SHAPE;
    int max_seq = tc->max_seq_len < dc->max_seq_len ? tc->max_seq_len : dc->max_seq_len;
    if (prompt_len >= max_seq) return REF_ERR_SHAPE;
    int available = max_seq - prompt_len;
    int max_new = max_new_tokens < available ? max_new_tokens : available;
    memset(stats, 0, sizeof(*stats));
    *out_len = 0;
    *finish_reason = REF_FINISH_MAX_TOKENS;
    float min_gap = INFINITY;
    if (max_new == 0) {
        *finish_reason = REF_FINISH_CONTEXT_LIMIT;
        if (out_min_gap) *out_min_gap = min_gap;
        return REF_OK;
    }
    int64_t V = tc->vocab_size;
    int K = num_draft_tokens;
    int det = ref_is_deterministic(s);
    ref_rng rng;
    ref_rng_seed_u64(&rng, seed);
    ref_kv *tkv = ref_kv_create(tm, tc->max_seq_len), *dkv = ref_kv_create(dm, dc->max_seq_len);
    float *tlog = (float *)malloc(sizeof(float) * (size_t)(prompt_len * V));
    float *dlog = (float *)malloc(sizeof(float) * (size_t)(prompt_len * V));
    float *target_next = (float *)malloc(sizeof(float) * (size_t)V);
    float *draft_next = (float *)malloc(sizeof(float) * (size_t)V);
    float *dist = (float *)malloc(sizeof(float) * (size_t)(K * V));
    float *vlog = (float *)malloc(sizeof(float) * (size_t)((K + 1) * V));
    float *pt = (float *)malloc(sizeof(float) * (size_t)V);
    float *res = (float *)malloc(sizeof(float) * (size_t)V);
    float *scratch = (float *)malloc(sizeof(float) * (size_t)((K + 1) * V));
    uint32_t *props = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)K);
    uint32_t *tin = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)(K + 1));
    int st = ref_forward(tm, tkv, prompt, prompt_len, 0, tlog, NULL, nt);
    if (!st) st = ref_forward(dm, dkv, prompt, prompt_len, 0, dlog, NULL, nt);
    if (!st) {
        memcpy(target_next, tlog + (int64_t)(prompt_len - 1) * V, sizeof(float) * (size_t)V);
        memcpy(draft_next, dlog + (int64_t)(prompt_len - 1) * V, sizeof(float) * (size_t)V);
    }
    free(tlog);
    free(dlog);
    int have_target_next = 1, pending = -1, n_out = 0;
    while (st == REF_OK && n_out < max_new) {
        int remaining = max_new - n_out;
        int count = K < remaining ? K : remaining;
        int committed = prompt_len + n_out;
        int tbase = tkv->len, dbase = dkv->len; /* snapshots (restore = index rewind) */
        (void)committed;
        int np = 0;
        ref_round rr;
        round_begin(&rr, n_out, &rng);
        for (int pi = 0; pi < count; pi++) {
            if (det) {
                float gp = top2_gap(draft_next, V);
                if (gp < min_gap) min_gap = gp;
                round_margin_logit(&rr, gp);
            }
            if ((st = ref_probabilities(s, draft_next, V, dist + (int64_t)pi * V))) break;
            round_margin_filter(&rr);
            uint32_t tok;
            float cmp = INFINITY;
            if ((st = ref_sample_probabilities(s, &rng, dist + (int64_t)pi * V, V, &tok, NULL, &cmp))) break;
            if (!det) round_margin_prob(&rr, cmp);
            props[np++] = tok;
            stats->draft_tokens_proposed++;
            if (tok == EOS_ID) break;
            if ((st = ref_forward(dm, dkv, &tok, 1, dkv->len, draft_next, NULL, nt))) break;
            stats->draft_decode_forwards++;
        }
        if (st) break;
        int hp = pending >= 0, nin = 0;
        if (hp) tin[nin++] = (uint32_t)pending;
        for (int i = 0; i < np; i++) tin[nin++] = props[i];
        if ((st = ref_forward(tm, tkv, tin, nin, tbase, vlog, NULL, nt))) break;
        stats->rounds++;
        stats->target_decode_forwards++;
        pending = -1;
        int rejected = 0, done = 0;
        rr.proposed = np;
        for (int i = 0; i < np; i++) {
            const float *tl = (hp || i > 0) ? vlog + (int64_t)(i - (hp ? 0 : 1)) * V : target_next;
            if (!hp && i == 0 && !have_target_next) { st = REF_ERR_CONFIG; break; }
            if (det) {
                float gp = top2_gap(tl, V);
                if (gp < min_gap) min_gap = gp;
                round_margin_logit(&rr, gp);
            }
            if ((st = ref_probabilities(s, tl, V, pt))) break;
            round_margin_filter(&rr);
            int acc = 0, drew = 0;
            float ratio = 0.0f, u = 0.0f;
            ref_accept_proposal(s, &rng, props[i], dist + (int64_t)i * V, pt, V, &acc, &ratio, &u, &drew);
            if (drew) round_margin_prob(&rr, fabsf(ratio - u));
            top_candidates(pt, V, 5, n_out);
            if (acc) {
                rr.accepted++;
                stats->draft_tokens_accepted++;
                if (props[i] == EOS_ID) {
                    *finish_reason = REF_FINISH_EOS;
                    done = 1;
                    break;
                }
                out_tokens[n_out++] = props[i];
                if (n_out == max_new) {
                    done = 1;
                    break;
                }
                continue;
            }
            rejected = 1;
            uint32_t repl;
            if (det) {
                if ((st = ref_sample_probabilities(s, &rng, pt, V, &repl, NULL, NULL))) break;
            } else {
                float cmr = INFINITY;
                if ((st = ref_residual(pt, dist + (int64_t)i * V, V, res))) break;
                if ((st = ref_sample_probabilities(s, &rng, res, V, &repl, NULL, &cmr))) break;
                round_margin_prob(&rr, cmr);
            }
            tkv->len = tbase; /* target_cache.restore */
            dkv->len = dbase; /* draft_cache.restore */
            int treplay = hp + i;
            if (treplay > 0 && (st = ref_forward(tm, tkv, tin, treplay, tbase, scratch, NULL, nt))) break;
            if (i > 0) {
                if ((st = ref_forward(dm, dkv, props, i, dbase, scratch, NULL, nt))) break;
                stats->draft_decode_forwards++;
            }
            if (repl == EOS_ID) {
                *finish_reason = REF_FINISH_EOS;
                done = 1;
                break;
            }
            out_tokens[n_out++] = repl;
            if ((st = ref_forward(dm, dkv, &repl, 1, dkv->len, draft_next, NULL, nt))) break;
            stats->draft_decode_forwards++;
            pending = (int)repl;
            break;
        }
        if (st) break;
        if (done || rejected || n_out == max_new) round_end(&rr, n_out, &rng);
        if (done) break;
        if (rejected) {
            have_target_next = 0;
            continue;
        }
        if (n_out == max_new) break;
        /* every proposal accepted: bonus from the row after the last proposal */
        const float *bl = vlog + (int64_t)(np - (hp ? 0 : 1)) * V;
        if (det) {
            float gp = top2_gap(bl, V);
            if (gp < min_gap) min_gap = gp;
            round_margin_logit(&rr, gp);
        }
        if ((st = ref_probabilities(s, bl, V, pt))) break;
        round_margin_filter(&rr);
        top_candidates(pt, V, 5, n_out);
        uint32_t bonus;
        float cmb = INFINITY;
        if ((st = ref_sample_probabilities(s, &rng, pt, V, &bonus, NULL, &cmb))) break;
        if (!det) round_margin_prob(&rr, cmb);
        if (bonus == EOS_ID) {
            *finish_reason = REF_FINISH_EOS;
            round_end(&rr, n_out, &rng);
            break;
        }
        out_tokens[n_out++] = bonus;
        round_end(&rr, n_out, &rng);
        if ((st = ref_forward(dm, dkv, &bonus, 1, dkv->len, draft_next, NULL, nt))) break;
        stats->draft_decode_forwards++;
        pending = (int)bonus;
        have_target_next = 0;
    }
    if (st == REF_OK) {
        if (n_out == available && *finish_reason == REF_FINISH_MAX_TOKENS)
            *finish_reason = REF_FINISH_CONTEXT_LIMIT;
        stats->draft_tokens_rejected = stats->draft_tokens_proposed - stats->draft_tokens_accepted;
        if (stats->draft_tokens_rejected < 0) stats->draft_tokens_rejected = 0;
    }
    *out_len = n_out;
    if (out_min_gap) *out_min_gap = min_gap;
    free(target_next);
    free(draft_next);
    free(dist);
    free(vlog);
    free(pt);
    free(res);
    free(scratch);
    free(props);
    free(tin);
    ref_kv_free(tkv);
    ref_kv_free(dkv);
    return st;
}

/* InferenceEngine plain decode (engine.rs generate path): sample, append, one-token forward. */
int ref_plain_generate(const ref_model *m, const uint32_t *prompt, int prompt_len,
                       int max_new_tokens, const ref_sampler *s, uint64_t seed, int nt,
                       uint32_t *out_tokens, int *out_len, int *finish_reason) {
    const ref_config *c = &m->cfg;
    if (prompt_len <= 0 || prompt_len >= c->max_seq_len) return REF_ERR_SHAPE;
    int available = c->max_seq_len - prompt_len;
    int max_new = max_new_tokens < available ? max_new_tokens : available;
    int64_t V = c->vocab_size;
    ref_rng rng;
    ref_rng_seed_u64(&rng, seed);
    ref_kv *kv = ref_kv_create(m, c->max_seq_len);
    float *plog = (float *)malloc(sizeof(float) * (size_t)(prompt_len * V));
    float *p = (float *)malloc(sizeof(float) * (size_t)V);
    float *last = (float *)malloc(sizeof(float) * (size_t)V);
    int st = ref_forward(m, kv, prompt, prompt_len, 0, plog, NULL, nt);
    memcpy(last, plog + (int64_t)(prompt_len - 1) * V, sizeof(float) * (size_t)V);
    *finish_reason = REF_FINISH_MAX_TOKENS;
    int n = 0;
    while (st == REF_OK && n < max_new) {
        if ((st = ref_probabilities(s, last, V, p))) break;
        uint32_t tok;
        if ((st = ref_sample_probabilities(s, &rng, p, V, &tok, NULL, NULL))) break;
        if (tok == EOS_ID) {
            *finish_reason = REF_FINISH_EOS;
            break;
        }
        out_tokens[n++] = tok;
        if (n == max_new) break;
        if ((st = ref_forward(m, kv, &tok, 1, kv->len, last, NULL, nt))) break;
    }
    if (st == REF_OK && n == available && *finish_reason == REF_FINISH_MAX_TOKENS)
        *finish_reason = REF_FINISH_CONTEXT_LIMIT;
    *out_len = n;
    free(plog);
    free(p);
    free(last);
    ref_kv_free(kv);
    return st;
}

/* ======================================================================== */
/* Latent-attention MoE decoder (benchmark config 5): every block is          */
/* x += MLA(norm1(x)) (nn/src/mla.rs:300-314,402-489; builder                */
/* model/src/model.rs:1094-1156) then x += MoE(norm2(x)) (nn/src/moe.rs:     */
/* 212-340, top_k_gating :361-406, SharedExpertPath :127-178).  The MLA      */
/* reconstructs K_nope = up_k(c_kv) and V = up_v(c_kv) over the whole cache, */
/* as the reference does; the device path absorbs up_k / up_v instead.      */
/* ======================================================================== */

enum { X_NORM1, X_QP, X_KVA, X_KVN, X_UPK, X_UPV, X_KRP, X_OP, X_NORM2, X_ROUTER, X_FIXED };

struct ref_lat {
    ref_lat_config cfg;
    int per_layer, n_tensors;
    ref_tensor *t;
    float *rope_cos, *rope_sin; /* [max_seq_len, rope_dim/2] (MLA's own RopeCache) */
};

struct ref_lat_kv {
    const ref_lat *m;
    int n_layers, capacity, len;
    float **ckv, **kr; /* per layer [capacity, latent], [capacity, rope] (cache-rounded values) */
};

static int lat_id(const ref_lat *m, int l, int which) { return 1 + l * m->per_layer + which; }
static int lat_expert_id(const ref_lat *m, int l, int e, int part) {
    return 1 + l * m->per_layer + X_FIXED + 3 * e + part; /* part: 0 gate, 1 up, 2 down */
}
static int lat_final_id(const ref_lat *m) { return 1 + m->cfg.n_layers * m->per_layer; }

ref_lat *ref_lat_create(const ref_lat_config *c) {
    if (c->vocab_size <= 0 || c->hidden_dim <= 0 || c->n_layers <= 0 || c->n_heads <= 0 ||
        c->max_seq_len <= 0 || c->latent_dim <= 0 || c->rope_dim <= 0 || (c->rope_dim & 1) ||
        c->nope_dim <= 0 || c->v_dim <= 0 || c->n_experts < 2 || c->top_k < 1 ||
        c->top_k > c->n_experts || c->expert_dim <= 0 || c->n_shared < 0)
        return NULL;
    ref_lat *m = (ref_lat *)calloc(1, sizeof(ref_lat));
    m->cfg = *c;
    m->per_layer = X_FIXED + 3 * (c->n_experts + c->n_shared);
    m->n_tensors = 2 + c->n_layers * m->per_layer + (c->untied_lm_head ? 1 : 0);
    m->t = (ref_tensor *)calloc((size_t)m->n_tensors, sizeof(ref_tensor));
    int64_t H = c->hidden_dim, h = c->n_heads, D = c->expert_dim;
    char nm[96];
    set_info(&m->t[0], "embedding.weight", c->vocab_size, H, REF_T_EMBED);
    for (int l = 0; l < c->n_layers; l++) {
#define XT(which, suffix, r, cc, k)                                                                \
    snprintf(nm, sizeof(nm), "blocks.%d.%s", l, suffix);                                           \
    set_info(&m->t[lat_id(m, l, which)], nm, r, cc, k);
        XT(X_NORM1, "norm1.weight", 1, H, REF_T_NORM)
        XT(X_QP, "mla.q_proj.weight", h * (c->nope_dim + c->rope_dim), H, REF_T_LINEAR)
        XT(X_KVA, "mla.kv_a_proj.weight", c->latent_dim, H, REF_T_LINEAR)
        XT(X_KVN, "mla.kv_a_norm.weight", 1, c->latent_dim, REF_T_NORM)
        XT(X_UPK, "mla.up_k.weight", h * c->nope_dim, c->latent_dim, REF_T_LINEAR)
        XT(X_UPV, "mla.up_v.weight", h * c->v_dim, c->latent_dim, REF_T_LINEAR)
        XT(X_KRP, "mla.k_rope_proj.weight", c->rope_dim, H, REF_T_LINEAR)
        XT(X_OP, "mla.o_proj.weight", H, h * c->v_dim, REF_T_LINEAR)
        XT(X_NORM2, "norm2.weight", 1, H, REF_T_NORM)
        XT(X_ROUTER, "ffn.router.weight", c->n_experts, H, REF_T_LINEAR)
#undef XT
        for (int e = 0; e < c->n_experts + c->n_shared; e++) {
            const char *grp = e < c->n_experts ? "experts" : "shared_experts";
            int ei = e < c->n_experts ? e : e - c->n_experts;
            snprintf(nm, sizeof(nm), "blocks.%d.ffn.%s.%d.w_gate.weight", l, grp, ei);
            set_info(&m->t[lat_expert_id(m, l, e, 0)], nm, D, H, REF_T_LINEAR);
            snprintf(nm, sizeof(nm), "blocks.%d.ffn.%s.%d.w_up.weight", l, grp, ei);
            set_info(&m->t[lat_expert_id(m, l, e, 1)], nm, D, H, REF_T_LINEAR);
            snprintf(nm, sizeof(nm), "blocks.%d.ffn.%s.%d.w_down.weight", l, grp, ei);
            set_info(&m->t[lat_expert_id(m, l, e, 2)], nm, H, D, REF_T_LINEAR);
        }
    }
    set_info(&m->t[lat_final_id(m)], "final_norm.weight", 1, H, REF_T_NORM);
    /* LmHead::untied_with_qat (model.rs:239-248): a [vocab, hidden] head of its own */
    if (c->untied_lm_head) set_info(&m->t[lat_final_id(m) + 1], "lm_head.weight", c->vocab_size, H, REF_T_EMBED);
    for (int i = 0; i < m->n_tensors; i++) {
        ref_tensor *t = &m->t[i];
        t->data = (float *)calloc((size_t)(t->rows * t->cols), sizeof(float));
        if (!t->data) {
            ref_lat_free(m);
            return NULL;
        }
        if (t->kind == REF_T_NORM)
            for (int64_t j = 0; j < t->rows * t->cols; j++) t->data[j] = 1.0f;
    }
    /* dedicated rope_dim-wide RoPE table (model.rs:1112-1118, rope_scaling.rs:6-11) */
    int half = c->rope_dim / 2, S = c->max_seq_len;
    m->rope_cos = (float *)malloc(sizeof(float) * (size_t)S * (size_t)half);
    m->rope_sin = (float *)malloc(sizeof(float) * (size_t)S * (size_t)half);
    for (int i = 0; i < half; i++) {
        float inv = (float)(1.0 / pow((double)c->rope_theta, 2.0 * (double)i / (double)c->rope_dim));
        for (int p = 0; p < S; p++) {
            float a = (float)p * inv;
            m->rope_cos[(size_t)p * half + i] = cosf(a);
            m->rope_sin[(size_t)p * half + i] = sinf(a);
        }
    }
    return m;
}

void ref_lat_free(ref_lat *m) {
    if (!m) return;
    for (int i = 0; i < m->n_tensors; i++) free(m->t[i].data);
    free(m->t);
    free(m->rope_cos);
    free(m->rope_sin);
    free(m);
}

int ref_lat_num_tensors(const ref_lat *m) { return m->n_tensors; }

int ref_lat_tensor_info(const ref_lat *m, int id, char *name, int name_cap, int64_t *rows, int64_t *cols,
                        int32_t *kind) {
    if (id < 0 || id >= m->n_tensors) return REF_ERR_SHAPE;
    snprintf(name, (size_t)name_cap, "%s", m->t[id].name);
    *rows = m->t[id].rows;
    *cols = m->t[id].cols;
    *kind = m->t[id].kind;
    return REF_OK;
}

/* Storage format of a tensor: experts in expert_format, MLA projections and the
   router in attn_format, the embedding and an untied head per lm_head_format. */
static int lat_format(const ref_lat *m, int id) {
    const ref_tensor *t = &m->t[id];
    if (t->kind == REF_T_EMBED) return m->cfg.lm_head_format == 1 ? REF_W_BF16 : REF_W_F32;
    if (id == 0 || id == lat_final_id(m)) return REF_W_F32;
    int w = (id - 1) % m->per_layer;
    return w >= X_FIXED ? m->cfg.expert_format : m->cfg.attn_format;
}

int ref_lat_set_tensor(ref_lat *m, int id, const float *raw) {
    if (id < 0 || id >= m->n_tensors) return REF_ERR_SHAPE;
    ref_tensor *t = &m->t[id];
    int64_t n = t->rows * t->cols;
    if (t->kind == REF_T_NORM) {
        memcpy(t->data, raw, sizeof(float) * (size_t)n);
        return REF_OK;
    }
    int fmt = lat_format(m, id);
    if (fmt == REF_W_F32) {
        memcpy(t->data, raw, sizeof(float) * (size_t)n);
    } else if (fmt == REF_W_BF16) {
        for (int64_t i = 0; i < n; i++) t->data[i] = ref_bf16_to_f32(ref_f32_to_bf16(raw[i]));
    } else if (fmt == REF_W_INT8_ROW) {
        int8_t *codes = (int8_t *)malloc((size_t)n);
        float *sc = (float *)malloc(sizeof(float) * (size_t)t->rows);
        ref_quantise_i8_rows(raw, t->rows, t->cols, codes, sc);
        for (int64_t r = 0; r < t->rows; r++)
            for (int64_t c = 0; c < t->cols; c++) t->data[r * t->cols + c] = (float)codes[r * t->cols + c] * sc[r];
        free(codes);
        free(sc);
    } else if (fmt == REF_W_INT4_G128) {
        if (t->cols % 128) return REF_ERR_SHAPE;
        int64_t ng = n / 128;
        uint8_t *packed = (uint8_t *)malloc((size_t)(n / 2));
        uint16_t *sh = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)ng);
        uint16_t *zh = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)ng);
        ref_quantise_i4_f16(raw, n, 128, packed, sh, zh);
        ref_dequantise_i4_f16(packed, n, 128, sh, zh, t->data);
        free(packed);
        free(sh);
        free(zh);
    } else {
        return REF_ERR_UNSUPPORTED;
    }
    return REF_OK;
}

int ref_lat_get_tensor(const ref_lat *m, int id, float *out) {
    if (id < 0 || id >= m->n_tensors) return REF_ERR_SHAPE;
    memcpy(out, m->t[id].data, sizeof(float) * (size_t)(m->t[id].rows * m->t[id].cols));
    return REF_OK;
}

/* Synthetic random-init model: tensor id i ~ N(0, std^2) on stream i, the
   router ~ N(0, 1/hidden_dim) so its logits on RMS-normalised inputs are about
   N(0, 1) (benchmark config 5), norms 1.  The device's synthetic init uses the
   same streams and scales. */
int ref_lat_init_synthetic(ref_lat *m, uint64_t seed, float std) {
    const float router_std = 1.0f / sqrtf((float)m->cfg.hidden_dim);
    for (int i = 0; i < m->n_tensors; i++) {
        ref_tensor *t = &m->t[i];
        if (t->kind == REF_T_NORM) continue;
        int64_t n = t->rows * t->cols;
        float *raw = (float *)malloc(sizeof(float) * (size_t)n);
        if (!raw) return REF_ERR_CONFIG;
        int is_router = i > 0 && i < lat_final_id(m) && (i - 1) % m->per_layer == X_ROUTER;
        ref_synth_fill(seed, (uint32_t)i, n, is_router ? router_std : std, raw);
        int st = ref_lat_set_tensor(m, i, raw);
        free(raw);
        if (st) return st;
    }
    return REF_OK;
}

ref_lat_kv *ref_lat_kv_create(const ref_lat *m, int capacity) {
    ref_lat_kv *kv = (ref_lat_kv *)calloc(1, sizeof(ref_lat_kv));
    kv->m = m;
    kv->n_layers = m->cfg.n_layers;
    kv->capacity = capacity;
    kv->ckv = (float **)calloc((size_t)kv->n_layers, sizeof(float *));
    kv->kr = (float **)calloc((size_t)kv->n_layers, sizeof(float *));
    for (int l = 0; l < kv->n_layers; l++) {
        kv->ckv[l] = (float *)calloc((size_t)capacity * (size_t)m->cfg.latent_dim, sizeof(float));
        kv->kr[l] = (float *)calloc((size_t)capacity * (size_t)m->cfg.rope_dim, sizeof(float));
        if (!kv->ckv[l] || !kv->kr[l]) {
            ref_lat_kv_free(kv);
            return NULL;
        }
    }
    return kv;
}

void ref_lat_kv_free(ref_lat_kv *kv) {
    if (!kv) return;
    for (int l = 0; l < kv->n_layers; l++) {
        if (kv->ckv) free(kv->ckv[l]);
        if (kv->kr) free(kv->kr[l]);
    }
    free(kv->ckv);
    free(kv->kr);
    free(kv);
}

int ref_lat_kv_truncate(ref_lat_kv *kv, int new_len) {
    if (new_len < 0 || new_len > kv->len) return REF_ERR_SHAPE;
    kv->len = new_len;
    return REF_OK;
}

static float lat_cache_round(const ref_lat *m, float v) {
    return m->cfg.kv_format == REF_KV_F16 ? ref_f16_to_f32(ref_f32_to_f16(v)) : v;
}

/* Synthetic latent cache: c_kv and k_rope ~ N(0, 1), streams per layer. */
int ref_lat_kv_fill_synthetic(ref_lat_kv *kv, uint64_t seed, int len) {
    const ref_lat *m = kv->m;
    if (len > kv->capacity) return REF_ERR_SHAPE;
    int lat = m->cfg.latent_dim, rd = m->cfg.rope_dim;
    for (int l = 0; l < m->cfg.n_layers; l++) {
        for (int64_t i = 0; i < (int64_t)len * lat; i++)
            kv->ckv[l][i] = lat_cache_round(m, ref_synth_normal(seed, 0x4C410000u + (uint32_t)(2 * l), (uint64_t)i));
        for (int64_t i = 0; i < (int64_t)len * rd; i++)
            kv->kr[l][i] = lat_cache_round(m, ref_synth_normal(seed, 0x4C410001u + (uint32_t)(2 * l), (uint64_t)i));
    }
    kv->len = len;
    return REF_OK;
}

/* RoPE of one rope_dim slice at position pos (rope.rs:107-126 on the MLA table). */
static void lat_rope(const ref_lat *m, float *v, int pos) {
    int half = m->cfg.rope_dim / 2;
    const float *c = m->rope_cos + (size_t)pos * half, *sn = m->rope_sin + (size_t)pos * half;
    for (int i = 0; i < half; i++) {
        float x1 = v[i], x2 = v[i + half];
        v[i] = x1 * c[i] - x2 * sn[i];
        v[i + half] = x1 * sn[i] + x2 * c[i];
    }
}

/*
 * top_k_gating (moe.rs:361-406): arg_sort_last_dim(descending), the first k
 * indices, softmax over the selected logits.  Equal logits keep the lower
 * expert index first (a stable descending sort).  idx/w are [rows][k].
 */
void ref_topk_gating(const float *logits, int rows, int E, int k, int32_t *idx, float *w) {
    for (int r = 0; r < rows; r++) {
        const float *l = logits + (int64_t)r * E;
        ranked_t *rk = (ranked_t *)malloc(sizeof(ranked_t) * (size_t)E);
        for (int e = 0; e < E; e++) rk[e] = (ranked_t){l[e], e};
        qsort(rk, (size_t)E, sizeof(ranked_t), cmp_ranked_desc);
        float mx = -INFINITY;
        for (int j = 0; j < k; j++) mx = fmaxf(mx, rk[j].v);
        float s = 0.0f;
        for (int j = 0; j < k; j++) {
            idx[(int64_t)r * k + j] = (int32_t)rk[j].i;
            w[(int64_t)r * k + j] = expf(rk[j].v - mx);
            s += w[(int64_t)r * k + j];
        }
        for (int j = 0; j < k; j++) w[(int64_t)r * k + j] /= s;
        free(rk);
    }
}

/* SwiGluFfn::forward (ffn.rs:29-37) of expert e on S rows of h (rows x H) -> y. */
static void lat_expert(const ref_lat *m, int l, int e, const float *h, int S, float *y, int nt) {
    int64_t H = m->cfg.hidden_dim, D = m->cfg.expert_dim;
    float *g = (float *)malloc(sizeof(float) * (size_t)(S * D));
    float *u = (float *)malloc(sizeof(float) * (size_t)(S * D));
    linear(h, S, H, m->t[lat_expert_id(m, l, e, 0)].data, D, g, nt);
    linear(h, S, H, m->t[lat_expert_id(m, l, e, 1)].data, D, u, nt);
    for (int64_t i = 0; i < (int64_t)S * D; i++) g[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
    linear(g, S, D, m->t[lat_expert_id(m, l, e, 2)].data, H, y, nt);
    free(g);
    free(u);
}

static void lat_block(const ref_lat *m, int l, float *x, int S, int pos0, ref_lat_kv *kv, int nt) {
    const ref_lat_config *c = &m->cfg;
    int64_t H = c->hidden_dim;
    int nh = c->n_heads, nope = c->nope_dim, rd = c->rope_dim, lat = c->latent_dim, vd = c->v_dim;
    int qw = nope + rd;
    float *h = (float *)malloc(sizeof(float) * (size_t)(S * H));
    rms_norm(x, S, H, m->t[lat_id(m, l, X_NORM1)].data, c->norm_eps, h);
    /* project (mla.rs:402-449) */
    float *q = (float *)malloc(sizeof(float) * (size_t)S * nh * qw);
    float *ck = (float *)malloc(sizeof(float) * (size_t)S * lat);
    float *ckn = (float *)malloc(sizeof(float) * (size_t)S * lat);
    float *kr = (float *)malloc(sizeof(float) * (size_t)S * rd);
    linear(h, S, H, m->t[lat_id(m, l, X_QP)].data, (int64_t)nh * qw, q, nt);
    linear(h, S, H, m->t[lat_id(m, l, X_KVA)].data, lat, ck, nt);
    rms_norm(ck, S, lat, m->t[lat_id(m, l, X_KVN)].data, c->norm_eps, ckn);
    linear(h, S, H, m->t[lat_id(m, l, X_KRP)].data, rd, kr, nt);
    for (int s = 0; s < S; s++) {
        for (int hh = 0; hh < nh; hh++) lat_rope(m, q + ((int64_t)s * nh + hh) * qw + nope, pos0 + s);
        lat_rope(m, kr + (int64_t)s * rd, pos0 + s);
        for (int i = 0; i < lat; i++) kv->ckv[l][(int64_t)(pos0 + s) * lat + i] = lat_cache_round(m, ckn[(int64_t)s * lat + i]);
        for (int i = 0; i < rd; i++) kv->kr[l][(int64_t)(pos0 + s) * rd + i] = lat_cache_round(m, kr[(int64_t)s * rd + i]);
    }
    /* attend (mla.rs:451-489): reconstruct K_nope and V over the whole cache */
    int T = pos0 + S;
    float *kn = (float *)malloc(sizeof(float) * (size_t)T * nh * nope);
    float *vv = (float *)malloc(sizeof(float) * (size_t)T * nh * vd);
    linear(kv->ckv[l], T, lat, m->t[lat_id(m, l, X_UPK)].data, (int64_t)nh * nope, kn, nt);
    linear(kv->ckv[l], T, lat, m->t[lat_id(m, l, X_UPV)].data, (int64_t)nh * vd, vv, nt);
    float scale = (float)(1.0 / sqrt((double)qw));
    float *att = (float *)malloc(sizeof(float) * (size_t)S * nh * vd);
#pragma omp parallel for num_threads(nt) schedule(static) collapse(2)
    for (int hh = 0; hh < nh; hh++)
        for (int s = 0; s < S; s++) {
            const float *qq = q + ((int64_t)s * nh + hh) * qw;
            int lim = pos0 + s; /* causal: shift kv_len - q_len */
            float mx = -INFINITY, l_ = 0.0f;
            float *o = att + ((int64_t)s * nh + hh) * vd;
            for (int i = 0; i < vd; i++) o[i] = 0.0f;
            for (int t = 0; t <= lim; t++) {
                float sc = (dotf(qq, kn + ((int64_t)t * nh + hh) * nope, nope) +
                            dotf(qq + nope, kv->kr[l] + (int64_t)t * rd, rd)) * scale;
                float mnew = fmaxf(mx, sc);
                float a = mx == -INFINITY ? 0.0f : expf(mx - mnew);
                float p = expf(sc - mnew);
                l_ = l_ * a + p;
                const float *vr = vv + ((int64_t)t * nh + hh) * vd;
                for (int i = 0; i < vd; i++) o[i] = o[i] * a + p * vr[i];
                mx = mnew;
            }
            for (int i = 0; i < vd; i++) o[i] /= l_;
        }
    float *y = (float *)malloc(sizeof(float) * (size_t)(S * H));
    linear(att, S, (int64_t)nh * vd, m->t[lat_id(m, l, X_OP)].data, H, y, nt);
    for (int64_t i = 0; i < (int64_t)S * H; i++) x[i] += y[i];
    /* MoE FFN (moe.rs:212-340) */
    rms_norm(x, S, H, m->t[lat_id(m, l, X_NORM2)].data, c->norm_eps, h);
    int E = c->n_experts, K = c->top_k;
    float *rl = (float *)malloc(sizeof(float) * (size_t)S * E);
    linear(h, S, H, m->t[lat_id(m, l, X_ROUTER)].data, E, rl, nt);
    int32_t *idx = (int32_t *)malloc(sizeof(int32_t) * (size_t)S * K);
    float *w = (float *)malloc(sizeof(float) * (size_t)S * K);
    ref_topk_gating(rl, S, E, K, idx, w);
    float *acc = (float *)calloc((size_t)(S * H), sizeof(float));
    float *ye = (float *)malloc(sizeof(float) * (size_t)H);
    for (int s = 0; s < S; s++) {
        /* routed: dispatch-weighted sum over experts in index order (unselected add 0) */
        for (int e = 0; e < E; e++) {
            float we = 0.0f;
            int sel = 0;
            for (int j = 0; j < K; j++)
                if (idx[(int64_t)s * K + j] == e) {
                    we = w[(int64_t)s * K + j];
                    sel = 1;
                }
            if (!sel) continue;
            lat_expert(m, l, e, h + (int64_t)s * H, 1, ye, 1);
            for (int64_t i = 0; i < H; i++) acc[(int64_t)s * H + i] += ye[i] * we;
        }
        /* shared experts, summed in order, then added to the routed output */
        if (c->n_shared > 0) {
            float *sh = (float *)calloc((size_t)H, sizeof(float));
            for (int e = 0; e < c->n_shared; e++) {
                lat_expert(m, l, E + e, h + (int64_t)s * H, 1, ye, 1);
                for (int64_t i = 0; i < H; i++) sh[i] = e == 0 ? ye[i] : sh[i] + ye[i];
            }
            for (int64_t i = 0; i < H; i++) acc[(int64_t)s * H + i] += sh[i];
            free(sh);
        }
    }
    for (int64_t i = 0; i < (int64_t)S * H; i++) x[i] += acc[i];
    free(h); free(q); free(ck); free(ckn); free(kr); free(kn); free(vv); free(att); free(y);
    free(rl); free(idx); free(w); free(acc); free(ye);
}

int ref_lat_forward(const ref_lat *m, ref_lat_kv *kv, const uint32_t *ids, int S, int offset, float *logits,
                    float *hidden, int nt) {
    const ref_lat_config *c = &m->cfg;
    if (S <= 0 || offset + S > c->max_seq_len) return REF_ERR_SHAPE;
    if (!kv || offset > kv->len || offset + S > kv->capacity) return REF_ERR_SHAPE;
    int64_t H = c->hidden_dim, V = c->vocab_size;
    for (int s = 0; s < S; s++)
        if ((int64_t)ids[s] >= V) return REF_ERR_SHAPE;
    kv->len = offset;
    float *x = (float *)malloc(sizeof(float) * (size_t)(S * H));
    const float *emb = m->t[0].data;
    for (int s = 0; s < S; s++) memcpy(x + s * H, emb + (int64_t)ids[s] * H, sizeof(float) * (size_t)H);
    for (int l = 0; l < c->n_layers; l++) lat_block(m, l, x, S, offset, kv, nt);
    kv->len = offset + S;
    float *hn = (float *)malloc(sizeof(float) * (size_t)(S * H));
    rms_norm(x, S, H, m->t[lat_final_id(m)].data, c->norm_eps, hn);
    if (hidden) memcpy(hidden, hn, sizeof(float) * (size_t)(S * H));
    if (logits) linear(hn, S, H, c->untied_lm_head ? m->t[lat_final_id(m) + 1].data : emb, V, logits, nt);
    free(hn);
    free(x);
    return REF_OK;
}
