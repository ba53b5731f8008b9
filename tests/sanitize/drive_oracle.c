/* Sanitizer driver of the CPU oracle (oracle/refcpu.c), built with AddressSanitizer and
   UndefinedBehaviorSanitizer by tests/sanitize/Makefile.  It runs every oracle entry
   point the tests use on small inputs, including the edge cases (top-k / top-p filters,
   ragged proposal counts, zero-mass residuals, bonus rows, context limits) so that an
   out-of-bounds access or undefined operation in the checker aborts the run. */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../oracle/refcpu.h"

#define CHECK(x)                                                        \
    do {                                                                \
        if (!(x)) {                                                     \
            fprintf(stderr, "check failed: %s (line %d)\n", #x, __LINE__); \
            exit(1);                                                    \
        }                                                               \
    } while (0)

static void sampler_and_acceptance(void) {
    ref_rng r;
    ref_rng_seed_u64(&r, 42);
    for (int i = 0; i < 100; i++) (void)ref_rng_next_f32(&r);
    ref_rng_set_pos(&r, 7);
    (void)ref_rng_word_f32(42, 1000);
    const int B = 4, K = 3;
    const int64_t V = 1000;
    float *target = malloc(sizeof(float) * B * (K + 1) * V), *draft = malloc(sizeof(float) * B * K * V);
    ref_synth_fill(1, 0, (int64_t)B * (K + 1) * V, 3.0f, target);
    ref_synth_fill(1, 1, (int64_t)B * K * V, 3.0f, draft);
    uint32_t toks[12];
    ref_synth_tokens(1, 2, B * K, (uint32_t)V, toks);
    int32_t np[4] = {3, 0, 2, 1};
    uint64_t seeds[4] = {1, 2, 3, 4}, offs[4] = {0, 5, 9, 100};
    ref_accept_result res[4];
    ref_sampler samplers[5] = {{1, 1.0f, 0, 1.0f}, {0, 0.8f, 0, 1.0f}, {0, 0.7f, 50, 0.9f}, {0, 1.0f, 1, 0.5f},
                               {0, 1.3f, 2000, 0.999f}};
    for (int s = 0; s < 5; s++)
        for (int bonus = 0; bonus < 2; bonus++) {
            CHECK(ref_accept_batch(B, K, V, target, K + 1, draft, toks, np, bonus, &samplers[s], seeds, offs, NULL,
                                   res) >= 0);
            CHECK(ref_accept_batch(B, K, V, target, K + 1, draft, toks, NULL, bonus, &samplers[s], seeds, NULL, NULL,
                                   res) >= 0);
        }
    float *p = malloc(sizeof(float) * V), *q = malloc(sizeof(float) * V), *res_p = malloc(sizeof(float) * V);
    CHECK(ref_probabilities(&samplers[2], target, V, p) == 0);
    (void)ref_last_topp_margin();
    (void)ref_last_topk_gap();
    CHECK(ref_validate_probabilities(p, V) == 0);
    CHECK(ref_probabilities(&samplers[1], draft, V, q) == 0);
    (void)ref_residual(p, p, V, res_p); /* zero mass: an error status, no crash */
    CHECK(ref_residual(p, q, V, res_p) == 0);
    uint32_t tok;
    float draw, margin;
    CHECK(ref_sample_probabilities(&samplers[1], &r, p, V, &tok, &draw, &margin) == 0 && tok < V);
    int acc, drew;
    float ratio;
    CHECK(ref_accept_proposal(&samplers[1], &r, 3, q, p, V, &acc, &ratio, &draw, &drew) == 0);
    uint32_t ids[5];
    float probs[5];
    ref_top_candidates(p, V, 5, ids, probs);
    free(target);
    free(draft);
    free(p);
    free(q);
    free(res_p);
}

static void quantisers(void) {
    float w[512], back[512], sc[4], zr[4];
    uint8_t packed[256];
    uint16_t sh[4], zh[4];
    ref_synth_fill(3, 0, 512, 0.1f, w);
    w[5] = 0.0f;
    CHECK(ref_quantise_i4(w, 512, 128, packed, sc, zr) == 0);
    CHECK(ref_dequantise_i4(packed, 512, 128, sc, zr, back) == 0);
    CHECK(ref_quantise_i4_f16(w, 512, 128, packed, sh, zh) == 0);
    CHECK(ref_dequantise_i4_f16(packed, 512, 128, sh, zh, back) == 0);
    int8_t codes[512];
    float rs[4];
    CHECK(ref_quantise_i8_rows(w, 4, 128, codes, rs) == 0);
    uint16_t kvs;
    CHECK(ref_quantise_kv_row(w, 128, codes, &kvs) == 0);
    for (int i = 0; i < 70000; i += 7) (void)ref_f16_to_f32(ref_f32_to_f16((float)i * 0.37f - 9000.0f));
    (void)ref_bf16_to_f32(ref_f32_to_bf16(3.14159f));
}

static ref_model *tiny_model(int wfmt, int kvfmt, int heads, uint64_t seed) {
    ref_config c = {512, 128, 256, 2, 4, 2, 64, 10000.0f, 1e-5f, heads, wfmt, wfmt == REF_W_F32 ? 0 : 1, kvfmt};
    ref_model *m = ref_model_create(&c);
    CHECK(m != NULL);
    CHECK(ref_model_init_synthetic(m, seed, 0.05f) == 0);
    return m;
}

static void models_and_engines(void) {
    const int fmts[3][2] = {{REF_W_F32, REF_KV_F32}, {REF_W_INT4_G128, REF_KV_INT8}, {REF_W_INT8_ROW, REF_KV_F16}};
    for (int f = 0; f < 3; f++) {
        ref_model *m = tiny_model(fmts[f][0], fmts[f][1], 3, 5 + f);
        ref_kv *kv = ref_kv_create(m, 64);
        uint32_t ids[64];
        ref_synth_tokens(5, 0, 64, 512, ids);
        float *logits = malloc(sizeof(float) * 24 * 512), *hidden = malloc(sizeof(float) * 24 * 128);
        CHECK(ref_forward(m, kv, ids, 20, 0, logits, hidden, 2) == 0);
        CHECK(ref_kv_truncate(kv, 12) == 0);
        CHECK(ref_forward(m, kv, ids + 12, 4, 12, logits, hidden, 2) == 0);
        CHECK(ref_forward_layers(m, kv, ids + 16, 2, 16, 1, 1, logits, 2) == 0);
        CHECK(ref_mtp_head(m, 1, hidden, ids, 2, logits, 2) == 0);
        CHECK(ref_kv_fill_synthetic(kv, 9, 40) == 0);
        ref_kv_free(kv);
        uint32_t out[40];
        int len, fin;
        ref_spec_stats st;
        float gap;
        ref_round rounds[64];
        int nr = 0;
        uint32_t cids[40 * 5];
        float cps[40 * 5];
        ref_set_round_sink(rounds, 64, &nr);
        ref_set_candidate_sink(cids, cps, 40);
        ref_sampler g = {1, 1.0f, 0, 1.0f}, t = {0, 0.7f, 50, 0.9f};
        CHECK(ref_mtp_generate(m, ids, 8, 30, 3, &g, 0, 2, out, &len, &fin, &st, &gap) == 0);
        CHECK(ref_mtp_generate(m, ids, 8, 30, 2, &t, 11, 2, out, &len, &fin, &st, &gap) == 0);
        CHECK(ref_mtp_generate(m, ids, 60, 30, 3, &g, 0, 2, out, &len, &fin, &st, &gap) == 0); /* context limit */
        ref_model *d = tiny_model(fmts[f][0], fmts[f][1], 0, 50 + f);
        CHECK(ref_spec_generate(m, d, ids, 8, 30, 3, &g, 0, 2, out, &len, &fin, &st, &gap) == 0);
        CHECK(ref_spec_generate(m, d, ids, 8, 30, 2, &t, 3, 2, out, &len, &fin, &st, &gap) == 0);
        CHECK(ref_plain_generate(m, ids, 8, 20, &t, 3, 2, out, &len, &fin) == 0);
        ref_set_round_sink(NULL, 0, NULL);
        ref_set_candidate_sink(NULL, NULL, 0);
        ref_model_free(d);
        ref_model_free(m);
        free(logits);
        free(hidden);
    }
}

static void latent_moe(void) {
    ref_lat_config c = {512, 256, 2, 4, 64, 10000.0f, 1e-6f, 64, 32, 32, 32, 8, 2, 128, 1,
                        REF_W_INT4_G128, REF_W_INT8_ROW, 1, REF_KV_F16};
    ref_lat *m = ref_lat_create(&c);
    CHECK(m != NULL);
    CHECK(ref_lat_init_synthetic(m, 3, 0.05f) == 0);
    ref_lat_kv *kv = ref_lat_kv_create(m, 64);
    uint32_t ids[16];
    ref_synth_tokens(3, 0, 16, 512, ids);
    float *logits = malloc(sizeof(float) * 16 * 512), *hidden = malloc(sizeof(float) * 16 * 256);
    CHECK(ref_lat_forward(m, kv, ids, 12, 0, logits, hidden, 2) == 0);
    CHECK(ref_lat_kv_truncate(kv, 6) == 0);
    CHECK(ref_lat_forward(m, kv, ids + 6, 4, 6, logits, hidden, 2) == 0);
    CHECK(ref_lat_kv_fill_synthetic(kv, 4, 30) == 0);
    float gl[3 * 8];
    int32_t gi[3 * 2];
    float gw[3 * 2];
    ref_synth_fill(4, 1, 24, 1.0f, gl);
    ref_topk_gating(gl, 3, 8, 2, gi, gw);
    ref_lat_kv_free(kv);
    ref_lat_free(m);
    free(logits);
    free(hidden);
}

int main(void) {
    sampler_and_acceptance();
    quantisers();
    models_and_engines();
    latent_moe();
    printf("oracle sanitizer run: ok\n");
    return 0;
}
