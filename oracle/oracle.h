/*
 * CPU oracle for the prompt-lookup / W4A8 hot path.  TEST INFRASTRUCTURE ONLY.
 *
 * This is a C++ restatement of Classevelabs/rai's AVX2 CPU path (rai-infer),
 * written with the same AVX2/FMA/F16C intrinsic sequences, lane structure and
 * accumulation order, so that its f32 results are bit-identical to the
 * reference's AVX2 build.  It exists to check the HIP implementation and to
 * time the CPU baseline; nothing in the shipped library links, loads or calls
 * it.  Only tests, the smoke check and the bench's CPU-baseline leg use it.
 *
 * Parity notes (each pinned by tests under tests/):
 *   - MAX_GROUPS (gemm.rs:1167, 128) is a validation-time parameter here
 *     (ora_model_open's max_groups); the arithmetic is unchanged.
 *   - Greedy prompt-lookup acceptance (argmax == draft) is the T->0 limit of
 *     lookup.rs:359-403; the reference itself rejects T <= 1e-6.
 *   - Only the Llama-shaped capability subset is implemented (v1 headers, and
 *     v2 headers whose only capabilities are embed_scale, attn_scale and MoE).
 *
 * All functions return 0 on success and a negative code on failure.
 */
#ifndef RAI_ORACLE_H
#define RAI_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ora_model ora_model;
typedef struct ora_kv ora_kv;
typedef struct ora_lookup ora_lookup;
typedef struct ora_rng ora_rng;
typedef struct ora_spec ora_spec;

typedef struct ora_config {
  uint32_t hidden_size, num_layers, num_heads, num_kv_heads, head_dim;
  uint32_t intermediate_size, vocab_size, max_context;
  float rope_theta, norm_eps;
  uint32_t group_size, embed_group_size, version, tied;
  uint32_t num_experts, experts_per_token, norm_topk_prob;
  float embed_scale, attn_scale;
} ora_config;

typedef struct ora_metrics {
  int32_t accepted, drafted, produced, matched_ngram; /* matched_ngram 0 = none */
} ora_metrics;

void ora_set_threads(int n);
int ora_get_threads(void);
const char *ora_last_error(void);

/* ---- kernel-level (gemm.rs) ---- */
int ora_quantize_split(const float *x, int cols, int gs, int8_t *q_even,
                       int8_t *q_odd, float *scales);
int ora_input_sums(const float *x, int cols, int gs, float *sums);
int ora_w4a8_matvec(float *out, const uint8_t *nib, const uint8_t *params,
                    const float *x, int rows, int cols, int gs);
int ora_w4a8_matmul(float *out, const uint8_t *nib, const uint8_t *params,
                    const float *x, int rows, int cols, int m, int gs);
/* Per (token, row, group) integer lane sums: 12 int32 per group,
 * [0..8) = 64-column-chunk lanes (zero when the group has no 64 chunk),
 * [8..12) = trailing 32-column block lanes (zero when absent). */
int ora_w4a8_lane_sums(int32_t *out, const uint8_t *nib, const float *x,
                       int rows, int cols, int m, int gs);
int ora_tied_lm_head(float *logits, const float *hidden, const uint8_t *codes,
                     const uint8_t *params, int vocab, int hidden_size, int gs);
int ora_embed_lookup(float *out, int token, const uint8_t *codes,
                     const uint8_t *params, int vocab, int hidden_size, int gs);

/* ---- layer-level (layers.rs) ---- */
int ora_rms_norm(float *out, const float *x, const float *w, int n, float eps);
int ora_rms_norm_residual(float *normed, float *residual, const float *x,
                          const float *w, int n, float eps);
int ora_silu_mul(float *gate, const float *up, int n);
int ora_rope_tables(float *cos_t, float *sin_t, int head_dim, int max_ctx,
                    float theta);
int ora_rope_apply(float *heads, int num_heads, int head_dim, const float *cos_row,
                   const float *sin_row);
/* One query head over cached K/V rows k[t*hd], v[t*hd] for t in 0..=pos. */
int ora_attention_head(const float *q, const float *k, const float *v, int pos,
                       int head_dim, float scale, float *out);
float ora_expf(float x);
float ora_schraudolph(float x);

/* ---- sampler / lookup (sampler.rs, lookup.rs) ---- */
int64_t ora_argmax(const float *values, int64_t n);
/* returns 1 and fills {ngram, start, len} on a match, 0 when none */
int ora_find_ngram_draft(const int32_t *tokens, int64_t len, int64_t min_ngram,
                         int64_t max_ngram, int64_t max_draft, int64_t *match3);

/* ---- exact sampling (rand 0.8 StdRng, sampler.rs, speculative.rs) ---- */
/* One ChaCha block: key[8], 64-bit counter (words 12-13), 64-bit stream
 * (words 14-15), `rounds` rounds (20 for the RFC vectors, 12 for StdRng). */
int ora_chacha_block(const uint32_t *key, uint64_t counter, uint64_t stream, int rounds, uint32_t *out16);
/* StdRng::seed_from_u64(seed) (key == NULL) or from_seed(key) over `rounds`. */
int ora_rng_create(uint64_t seed, int rounds, const uint32_t *key, ora_rng **out);
void ora_rng_free(ora_rng *r);
uint32_t ora_rng_next_u32(ora_rng *r);
uint64_t ora_rng_next_u64(ora_rng *r);
float ora_rng_gen_f32(ora_rng *r);
double ora_rng_gen_f64(ora_rng *r);
/* The Standard f32 / f64 of one u32 / u64, as gen_f32 / gen_f64 apply it. */
float ora_standard_f32(uint32_t u);
double ora_standard_f64(uint64_t u);
void ora_rng_key(const ora_rng *r, uint32_t *key8);
int ora_softmax_probabilities(const float *logits, int n, float temperature, float *out);
int ora_sample_token(const float *logits, int n, float temperature, ora_rng *r, int *token);
/* lookup.rs:359-403 over verify logits [nd + 1][V] against draft[nd]. */
int ora_sampled_accept(const float *logits, int vocab, const int32_t *draft, int nd, float temperature,
                       ora_rng *r, int32_t *out, int *produced, int *accepted);

/* ---- model (format.rs, model.rs, kv_cache.rs) ---- */
int ora_model_open(const uint8_t *buf, size_t len, int max_groups, ora_model **out);
void ora_model_free(ora_model *m);
int ora_model_config(const ora_model *m, ora_config *out);
int ora_kv_create(const ora_model *m, int max_ctx, ora_kv **out);
void ora_kv_free(ora_kv *kv);
int ora_kv_truncate(ora_kv *kv, int len);
int ora_kv_filled(const ora_kv *kv, int layer);
/* One cached K (which = 0) or V (which = 1) row [head_dim] (kv_cache.rs:179-204). */
int ora_kv_read(const ora_kv *kv, int layer, int head, int pos, int which, float *out);
/* Positions 0..npos of one layer's K (which = 0) or V (1) from rows
 * [kv_head][npos][head_dim] (kv_cache.rs:143-173 in bulk); filled = npos. */
int ora_kv_import(ora_kv *kv, int layer, int which, const float *rows, int npos);
/* route_experts (layers.rs:1808-1870) for one token: experts[k] / weights[k]
 * for k < topk (-1 / 0 past the selection). */
int ora_route_experts(const float *router, const float *x, int hidden, int num_experts, int topk,
                      int norm_topk_prob, int32_t *experts, float *weights);
int ora_embed_token(const ora_model *m, int token, float *out);
int ora_forward_from_hidden(const ora_model *m, ora_kv *kv, float *hidden, int pos,
                            int store_kv);
int ora_forward_batch(const ora_model *m, ora_kv *kv, float *hiddens,
                      const int32_t *positions, int batch);
int ora_hidden_to_logits(const ora_model *m, const float *hidden, float *logits);
int ora_hidden_to_logits_batch(const ora_model *m, const float *hiddens,
                               float *logits, int batch);

/* ---- decoders ---- */
int ora_lookup_create(const ora_model *m, int max_ctx, ora_lookup **out);
void ora_lookup_free(ora_lookup *d);
int ora_lookup_prefill(ora_lookup *d, const int32_t *prompt, int n, int *pos_out);
int ora_lookup_step_greedy(ora_lookup *d, int pos, const int32_t *context, int len,
                           int max_draft, int min_ngram, int max_ngram,
                           int32_t *out_tokens, ora_metrics *metrics);
int ora_lookup_step_sampled(ora_lookup *d, int pos, const int32_t *context, int len, int max_draft,
                            int min_ngram, int max_ngram, float temperature, ora_rng *rng,
                            int32_t *out_tokens, ora_metrics *metrics);
int ora_lookup_kv_filled(const ora_lookup *d);
/* decode_one (lookup.rs:428-455) with argmax: embed `token` at `pos`,
 * forward, logits, argmax into *out. */
int ora_lookup_decode_one(ora_lookup *d, int pos, int token, int32_t *out);
/* The plain sampled step (run.rs:692-735): forward of `token` at `pos`, the
 * repetition penalty over ctx[0..len), sample_token with the config. */
int ora_lookup_decode_sample(ora_lookup *d, int pos, int token, const int32_t *ctx, int len, float temperature,
                             int64_t top_k, float top_p, float penalty, ora_rng *rng, int32_t *out);
/* apply_repetition_penalty (sampler.rs:185-199) over ctx[0..len), then
 * sample_token (sampler.rs:47-182) with the whole SamplerConfig. */
int ora_sample_plain(const float *logits, int n, const int32_t *ctx, int len, float temperature, int64_t top_k,
                     float top_p, float penalty, ora_rng *r, int *token);
/* SpeculativeDecoder (speculative.rs:79-391); temperature <= 1e-6 is the
 * greedy variant (argmax drafts, argmax acceptance). */
int ora_spec_create(const ora_model *draft, const ora_model *target, int max_ctx, ora_spec **out);
void ora_spec_free(ora_spec *d);
int ora_spec_prefill(ora_spec *d, const int32_t *prompt, int n, int *pos_out);
int ora_spec_step(ora_spec *d, int pos, int last_token, int draft_k, float temperature, ora_rng *rng,
                  int32_t *out_tokens, ora_metrics *metrics);
int ora_spec_accept(const float *target_logits, const float *draft_logits, int vocab, const int32_t *draft,
                    int k, float temperature, ora_rng *r, int32_t *out, int *produced, int *accepted);
/* Replace layer `layer`'s K (which = 0) or V (which = 1) rows with
 * rows[nkv][npos][head_dim] and set its watermark to npos (a decoder state
 * taken from another implementation, e.g. to time steps at a long context
 * without running the prefill on the CPU). */
int ora_lookup_import_kv(ora_lookup *d, int layer, int which, const float *rows, int npos);
/* Plain greedy decode: prefill prompt[0..n-1], then `steps` decode_one calls. */
int ora_greedy_generate(const ora_model *m, const int32_t *prompt, int n, int steps,
                        int max_ctx, int32_t *out_tokens);

#ifdef __cplusplus
}
#endif
#endif
