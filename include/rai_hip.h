/*
 * rai_hip.h -- C ABI of the MI355X (gfx950) prompt-lookup / W4A8 library.
 *
 * This library re-implements, for one MI355X GPU, the hot path of
 * Classevelabs/rai's `rai_infer` crate: prompt-lookup speculative decoding,
 * the (k+1)-token verify forward pass, greedy acceptance with KV rollback,
 * and the W4A8 GEMV/GEMM beneath them.  Each entry point below names the
 * reference interface it replaces (rai-infer/src/<file>:<line>).  A Rust
 * `extern "C"` crate can bind these symbols one-to-one.
 *
 * Conventions
 *   - Every function returns an rai_status (0 = RAI_OK).  On failure the
 *     thread's last error text is available from rai_last_error().  Where the
 *     reference panics on a shape/buffer violation (gemm.rs:1169-1213,
 *     layers.rs:1109-1168, kv_cache.rs:143-204), this ABI returns
 *     RAI_E_SHAPE / RAI_E_WATERMARK instead; where it returns anyhow::Err it
 *     returns the matching status.
 *   - Handles are opaque and owned by the library; free them with the
 *     matching *_free.  A handle is not re-entrant: one host thread at a time.
 *   - Token ids are uint32.  Sizes are size_t.  No torch types appear here.
 *   - Host-pointer entry points copy in/out and synchronise before returning.
 *     Device-pointer entry points (suffix _dev) take a hipStream_t passed as
 *     void* (NULL = the null stream) and are asynchronous.
 *   - Arithmetic is bit-identical to the reference's AVX2 path on the same
 *     inputs: integer accumulators, f32 outputs, logits and token streams.
 */
#ifndef RAI_HIP_H
#define RAI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum rai_status {
  RAI_OK = 0,
  RAI_E_ARG = -1,         /* invalid argument / configuration */
  RAI_E_SHAPE = -2,       /* buffer or dimension violation (reference: assert!) */
  RAI_E_FORMAT = -3,      /* malformed or hostile .raimodel file */
  RAI_E_OOM = -4,         /* host or device allocation failed */
  RAI_E_HIP = -5,         /* HIP runtime error */
  RAI_E_WATERMARK = -6,   /* KV store gap or read above the filled watermark */
  RAI_E_UNSUPPORTED = -7, /* a capability this build does not implement */
  RAI_E_IO = -8,          /* file could not be read */
  RAI_E_RANGE = -9        /* token id / position outside the model's range */
} rai_status;

typedef struct rai_model rai_model;
typedef struct rai_kv rai_kv;
typedef struct rai_lookup rai_lookup;
typedef struct rai_spec rai_spec;

/* ModelConfig (format.rs:162-265), the fields this build implements. */
typedef struct rai_model_config {
  uint32_t hidden_size, num_layers, num_heads, num_kv_heads, head_dim;
  uint32_t intermediate_size, vocab_size, max_context;
  float rope_theta, norm_eps;
  uint32_t group_size, embed_group_size, version;
  uint32_t tied;              /* 1 = lm_head tied to the 8-bit embedding */
  uint32_t num_experts;       /* 0 = dense MLP */
  uint32_t experts_per_token;
  uint32_t norm_topk_prob;
  float embed_scale, attn_scale; /* attn_scale is the effective multiplier */
} rai_model_config;

/* LookupConfig (lookup.rs:64-89).  temperature <= 1e-6 selects greedy
 * acceptance (argmax == draft), the T->0 limit of lookup.rs:359-403; above
 * it the step samples exactly as the reference does. */
typedef struct rai_lookup_config {
  size_t max_draft;   /* K */
  size_t max_ngram;
  size_t min_ngram;   /* >= 1 */
  float temperature;  /* > 1e-6: exact sampling (lookup.rs:359-403) from the
                         decoder's StdRng; <= 1e-6: greedy acceptance */
} rai_lookup_config;

/* SamplerConfig (sampler.rs:17-42) with the repetition penalty `rai run`
 * applies over the context (run.rs:720): temperature (<= 1e-6 or non-finite:
 * argmax), top_k (0 = off), top_p (1 = off; NaN = 1), repetition_penalty
 * (1 = off). */
typedef struct rai_sampler_config {
  float temperature;
  size_t top_k;
  float top_p;
  float repetition_penalty;
} rai_sampler_config;

/* SpeculativeConfig (speculative.rs:25-45): draft_k and the sampler's
 * temperature (top_k 0, top_p 1, no repetition penalty: the exact
 * configuration).  temperature <= 1e-6 selects the greedy variant (argmax
 * drafts, accepted while the target's argmax agrees), which the reference
 * refuses. */
typedef struct rai_spec_config {
  size_t draft_k;
  float temperature;
} rai_spec_config;

/* SpeculativeMetrics (speculative.rs:47-58). */
typedef struct rai_spec_metrics {
  size_t accepted, drafted, produced;
  float accept_rate;
} rai_spec_metrics;

/* LookupMatch (lookup.rs:91-109). */
typedef struct rai_lookup_match {
  size_t ngram, start, len;
} rai_lookup_match;

/* LookupMetrics (lookup.rs:112-119); matched_ngram == 0 means no match. */
typedef struct rai_lookup_metrics {
  size_t accepted, drafted, produced, matched_ngram;
  float accept_rate;
} rai_lookup_metrics;

/* Aggregate statistics of rai_lookup_generate (the `rai run` stats,
 * cli/run.rs:623-633). */
typedef struct rai_generate_stats {
  size_t prompt_tokens, generated, steps, steps_with_draft, drafted, accepted;
  double prefill_seconds, decode_seconds;
} rai_generate_stats;

/* ---------------------------------------------------------------- errors -- */
const char *rai_last_error(void);
/* HIP device the library runs on (reads HIP_VISIBLE_DEVICES semantics). */
int rai_device_info(char *name, size_t name_len, int *compute_units);

/* ----------------------------------------------------------------- model -- */
/* RaiModel::load (model.rs:97-181) + RaiModelFile::open (format.rs:557-637):
 * reads and validates the whole file with the reference's rules
 * (format.rs:1098-1521), then uploads it to HBM.  max_groups replaces the
 * reference's MAX_GROUPS = 128 (gemm.rs:1167); pass 0 for the reference value
 * 128, or a larger bound for group-32 models with K > 4096.  Device memory:
 * the file's bytes, RoPE tables, and for group-32 dense matrices a second
 * copy of their scale/zero parameters in 16-row tiles (about a fifth of the
 * quantized weight bytes), which the 2..64-token GEMVs read. */
int rai_model_open(const char *path, int max_groups, rai_model **out);
/* Same, from a caller-owned in-memory .raimodel image (copied). */
int rai_model_from_buffer(const void *data, size_t len, int max_groups, rai_model **out);
void rai_model_free(rai_model *model);
int rai_model_get_config(const rai_model *model, rai_model_config *out);
/* Bytes of quantized weights one decode step streams (linears + lm_head). */
int rai_model_weight_bytes(const rai_model *model, uint64_t *out);

/* --------------------------------------------------------------- KV cache -- */
/* RaiModel::create_kv_cache (model.rs:350) / KVCache::new (kv_cache.rs:232).
 * f32 [layer][kv_head][max_ctx][head_dim] in HBM, allocated up front. */
int rai_kv_create(rai_model *model, size_t max_ctx, rai_kv **out);
void rai_kv_free(rai_kv *kv);
/* KVCache::truncate (kv_cache.rs:300-304): filled = min(filled, len). */
int rai_kv_truncate(rai_kv *kv, size_t len);
/* KVCache::filled (kv_cache.rs:292). */
int rai_kv_filled(const rai_kv *kv, size_t layer, size_t *out);
/* KVCache::clear (kv_cache.rs:316). */
int rai_kv_clear(rai_kv *kv);
/* Copy one cached K or V row [head_dim] (kv_cache.rs:179-204 get_k/get_v);
 * which = 0 for K, 1 for V.  Reads at or above the watermark fail. */
int rai_kv_read(const rai_kv *kv, size_t layer, size_t head, size_t pos, int which, float *out);
/* get_k / get_v in bulk: rows [kv_head][npos][head_dim] of one layer for
 * positions 0..npos (npos <= filled), e.g. to hand a decoder state to
 * another implementation. */
int rai_kv_export(const rai_kv *kv, size_t layer, int which, float *out, size_t npos);
/* KVCache::store (kv_cache.rs:143-173, 257-265) in bulk, the inverse of
 * rai_kv_export: rows [kv_head][npos][head_dim] of one layer's K (which = 0)
 * or V (1) become positions 0..npos, and the layer's watermark becomes npos
 * (a state handed over from another implementation).  npos above the
 * cache's positions fails with RAI_E_RANGE. */
int rai_kv_import(rai_kv *kv, size_t layer, int which, const float *rows, size_t npos);

/* ---------------------------------------------------------- forward pass -- */
/* RaiModel::embed_token (model.rs:371-403). */
int rai_embed_token(rai_model *model, size_t token, float *out);
/* RaiModel::forward_from_hidden (model.rs:407-499); store_kv must be 1. */
int rai_forward_from_hidden(rai_model *model, rai_kv *kv, float *hidden, size_t pos, int store_kv);
/* RaiModel::forward_batch (model.rs:692-963): hiddens [batch][hidden] in/out,
 * positions strictly consecutive. */
int rai_forward_batch(rai_model *model, rai_kv *kv, float *hiddens, const size_t *positions,
                      size_t batch);
/* RaiModel::hidden_to_logits_into (model.rs:504-548). */
int rai_hidden_to_logits(rai_model *model, const float *hidden, float *logits);
/* RaiModel::hidden_to_logits_batch (model.rs:966-1033). */
int rai_hidden_to_logits_batch(rai_model *model, const float *hiddens, float *logits,
                               size_t batch);

/* ------------------------------------------------------- kernels (device) -- */
/* w4a8_matmul (gemm.rs:1774-1919); m == 1 is w4a8_matvec (gemm.rs:1336-1384).
 * out[t*rows + r], x[t*cols + c]; weights in the .raimodel linear layout:
 * nibbles [rows][cols/2] (low nibble = even column) and params
 * [rows][ceil(cols/gs)] x (f16 scale, f16 zero).  All pointers are device
 * pointers. */
int rai_w4a8_matmul_dev(float *out, const uint8_t *nibbles, const uint8_t *params,
                        const float *x, size_t rows, size_t cols, size_t m, size_t group_size,
                        void *stream);
/* One quantized linear on the device: QuantizedLinear (format.rs:361-367)
 * with device pointers to its nibbles [rows][cols/2] and params
 * [rows][ceil(cols/group_size)] x (f16 scale, f16 zero). */
typedef struct rai_qlinear {
  const uint8_t *nibbles;
  const uint8_t *params;
  size_t rows, cols, group_size;
} rai_qlinear;
/* w4a8_fused_qkv (gemm.rs:1386-1557): one input row x [cols] quantized once
 * and shared by the three projections; q_out [q.rows], k_out [k.rows],
 * v_out [v.rows], each equal to w4a8_matvec of its projection.  Each
 * projection is validated as w4a8_matvec's (RAI_E_SHAPE), and the three
 * must agree on cols and group_size ("Q/K column mismatch" etc.,
 * RAI_E_SHAPE).  Device pointers; synchronous on `stream`. */
int rai_w4a8_fused_qkv_dev(float *q_out, float *k_out, float *v_out, const rai_qlinear *q,
                           const rai_qlinear *k, const rai_qlinear *v, const float *x, void *stream);
/* w4a8_fused_gate_up (gemm.rs:1559-1703): the same for gate and up. */
int rai_w4a8_fused_gate_up_dev(float *gate_out, float *up_out, const rai_qlinear *gate,
                               const rai_qlinear *up, const float *x, void *stream);
/* Allocation-free variant of rai_w4a8_matmul_dev.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, arithmetic and results; the quantized activations live in
 * a fixed per-GPU scratch array held until the process ends (8 MiB),
 * so the call is asynchronous on `stream` and calls no allocator.  Limits:
 * m * cols <= 1048576 and m * ceil(cols / group_size) <= 65536, else
 * RAI_E_SHAPE.  Every call on one GPU shares that GPU's scratch: calls that
 * overlap in time on one GPU (other streams, other host threads) race. */
int rai_w4a8_matmul_noalloc_dev(float *out, const uint8_t *nibbles, const uint8_t *params,
                                const float *x, size_t rows, size_t cols, size_t m,
                                size_t group_size, void *stream);
/* Debug companion (no reference counterpart): the integer accumulators of
 * matvec_chunk_i8 (gemm.rs:458-525) per (token, row, group) as 12 int32:
 * [0..8) the 64-column-chunk lanes, [8..12) the trailing 32-column block. */
int rai_w4a8_lane_sums_dev(int32_t *out, const uint8_t *nibbles, const float *x, size_t rows,
                           size_t cols, size_t m, size_t group_size, void *stream);
/* Kernel timer (the role of the reference's gemm-bench, bin/gemm_bench.rs:9-77):
 * quantizes x once, then launches the W4A8 kernel `iters` times back to back
 * on its own stream between two HIP events; *avg_ms = elapsed / iters.
 * nibbles / params hold `copies` >= 1 back-to-back copies of the weights and
 * launch i reads copy i % copies, so that enough copies (together larger
 * than the GPU's last-level cache) make every launch stream its weights from
 * HBM as in a model step.  Device pointers. */
int rai_w4a8_time_dev(float *out, const uint8_t *nibbles, const uint8_t *params, const float *x,
                      size_t rows, size_t cols, size_t m, size_t group_size, size_t copies,
                      int iters, float *avg_ms);
/* Attention timer (no reference counterpart; the attention-side companion
 * of rai_w4a8_time_dev): the production attention of `m` tokens at
 * positions pos..pos+m-1 (m <= 64) over a K cache [nkv][cap][hd] and a
 * d-major V cache [nkv][hd][vstride] (vstride = cap rounded up to 64): one
 * full pass, then the score, softmax and PV launches each `iters` times back
 * to back between two HIP events; ms3 = the average milliseconds of each of
 * the three.  q is [m][nh*hd]; kc / vc hold `copies` back-to-back caches and
 * launch i reads copy i % copies (enough copies make every launch stream K
 * and V from HBM, as in a model step).  Device pointers. */
int rai_attention_time_dev(const float *q, const float *kc, const float *vc, size_t cap, size_t pos, size_t m,
                           size_t nh, size_t nkv, size_t hd, size_t copies, int iters, float *ms3);
/* Host-pointer convenience wrapper of rai_w4a8_matmul_dev (copies in/out). */
int rai_w4a8_matmul(float *out, const uint8_t *nibbles, const uint8_t *params, const float *x,
                    size_t rows, size_t cols, size_t m, size_t group_size);
/* tied_lm_head (gemm.rs:1981-2076), device pointers. */
int rai_tied_lm_head_dev(float *logits, const float *hidden, const uint8_t *codes,
                         const uint8_t *params, size_t vocab, size_t hidden_size,
                         size_t group_size, void *stream);
/* embed_lookup (gemm.rs:1926-1970), device pointers, one token. */
int rai_embed_lookup_dev(float *out, size_t token, const uint8_t *codes, const uint8_t *params,
                         size_t vocab, size_t hidden_size, size_t group_size, void *stream);

/* argmax (sampler.rs:201-208) of each of `rows` logit rows [rows][vocab]:
 * NaN counts as -inf, values compare by f32::total_cmp (-0 < +0), and the
 * last maximal index wins.  Device pointers; out[rows] uint32. */
int rai_argmax_dev(const float *logits, size_t rows, size_t vocab, uint32_t *out, void *stream);

/* ------------------------------------------------ layer kernels (device) -- */
/* rms_norm (layers.rs:154-183, 325-376) over m rows of n. */
int rai_rms_norm_dev(float *out, const float *x, const float *weight, size_t m, size_t n,
                     float eps, void *stream);
/* silu_mul_inplace (layers.rs:824-883) over m rows of n: gate = silu(gate)*up. */
int rai_silu_mul_dev(float *gate, const float *up, size_t m, size_t n, void *stream);
/* RoPETable::apply (layers.rs:643-726) of one position's cos/sin rows
 * ([head_dim/2] each) to heads [num_heads][head_dim], in place. */
int rai_rope_apply_dev(float *heads, size_t num_heads, size_t head_dim, const float *cos_row,
                       const float *sin_row, void *stream);
/* attention_head (layers.rs:1266-1452) for one query head over cached rows
 * k[t][head_dim], v[t][head_dim], t in 0..=pos (softcap disabled). */
int rai_attention_head_dev(float *out, const float *q, const float *k, const float *v, size_t pos,
                           size_t head_dim, float scale, void *stream);

/* -------------------------------------------- draft-model speculation -- */
/* SpeculativeDecoder::new (speculative.rs:79-110): both models must share
 * the vocabulary; the context is the smaller of both windows and max_ctx. */
int rai_spec_create(rai_model *draft, rai_model *target, size_t max_ctx, rai_spec **out);
void rai_spec_free(rai_spec *dec);
/* The `pub draft_kv` (which = 0) / `pub target_kv` (1) caches: borrowed. */
int rai_spec_kv(rai_spec *dec, int which, rai_kv **out);
/* StdRng::seed_from_u64(seed) for the sampled steps (new decoders: 0). */
int rai_spec_seed(rai_spec *dec, uint64_t seed);
/* SpeculativeDecoder::prefill (speculative.rs:112-171): both models over
 * prompt[0..n-1] (batched; bit-identical to the reference's token loop). */
int rai_spec_prefill(rai_spec *dec, const uint32_t *prompt, size_t n, size_t *pos_out);
/* SpeculativeDecoder::step (speculative.rs:180-391): writes metrics->produced
 * tokens (capacity >= draft_k + 1). */
int rai_spec_step(rai_spec *dec, size_t pos, uint32_t last_token, const rai_spec_config *cfg,
                  uint32_t *out_tokens, size_t out_cap, rai_spec_metrics *metrics);

/* ----------------------------------------------------- prompt-lookup path -- */
/* find_ngram_draft (lookup.rs:131-171), evaluated by the GPU search kernel.
 * *found = 0 when there is no match. */
int rai_find_ngram_draft(const uint32_t *tokens, size_t len, size_t min_ngram, size_t max_ngram,
                         size_t max_draft, rai_lookup_match *out, int *found);
/* LookupDecoder::new (lookup.rs:192-212). */
int rai_lookup_create(rai_model *model, size_t max_ctx, rai_lookup **out);
void rai_lookup_free(rai_lookup *dec);
/* The decoder's generator for exact sampling: rand::rngs::StdRng::
 * seed_from_u64(seed) (run.rs:345 seeds the `rng` passed to step).  A new
 * decoder starts from seed 0. */
int rai_lookup_seed(rai_lookup *dec, uint64_t seed);
/* n draws from a fresh StdRng::seed_from_u64(seed) on the device generator
 * (kinds[i]: 0 next_u32, 1 next_u64, 2 gen::<f32>, 3 gen::<f64>; out[i]
 * holds the value's bits).  No counterpart in the reference: it exposes the
 * generator the sampled steps use, for checking against other
 * implementations of rand 0.8's StdRng. */
int rai_std_rng_draws(uint64_t seed, const int *kinds, size_t n, uint64_t *out);
/* The decoder's `pub kv_cache` (lookup.rs:176): borrowed, do not free. */
int rai_lookup_kv(rai_lookup *dec, rai_kv **out);
/* LookupDecoder::prefill (lookup.rs:219-247): forward over prompt[0..n-1]. */
int rai_lookup_prefill(rai_lookup *dec, const uint32_t *prompt, size_t n, size_t *pos_out);
/* LookupDecoder::step (lookup.rs:260-425).  context[len-1] lives at pos.
 * Writes metrics->produced tokens into out_tokens (capacity >= max_draft+1). */
int rai_lookup_step(rai_lookup *dec, size_t pos, const uint32_t *context, size_t len,
                    const rai_lookup_config *cfg, uint32_t *out_tokens, size_t out_cap,
                    rai_lookup_metrics *metrics);
/* The `rai run --lookup-k` loop (cli/run.rs:517-633) without the tokenizer:
 * prefill, then steps until max_tokens are generated.  out_tokens receives
 * the generated ids (capacity >= max_tokens + max_draft). */
int rai_lookup_generate(rai_lookup *dec, const uint32_t *prompt, size_t n, size_t max_tokens,
                        const rai_lookup_config *cfg, uint32_t *out_tokens, size_t out_cap,
                        size_t *n_out, rai_generate_stats *stats);
/* The same loop without the prefill: steps from a decoder whose KV cache
 * holds context[0..len-1) (pos = len - 1), e.g. after rai_lookup_prefill, or
 * after rai_kv_truncate back to a prefilled prompt.  stats->prefill_seconds
 * is 0. */
int rai_lookup_decode(rai_lookup *dec, const uint32_t *context, size_t len, size_t pos,
                      size_t max_tokens, const rai_lookup_config *cfg, uint32_t *out_tokens,
                      size_t out_cap, size_t *n_out, rai_generate_stats *stats);
/* Plain greedy decode (sampler.rs:61-64 argmax after decode_one,
 * lookup.rs:428-455): prefill, then `steps` single-token steps (the `rai run`
 * loop without speculation at temperature 0, run.rs:640-735).  Also the
 * token-identity check of the lookup decoder. */
int rai_greedy_generate(rai_lookup *dec, const uint32_t *prompt, size_t n, size_t steps,
                        uint32_t *out_tokens);
/* The same decode loop from a prefilled state: context[len - 1] is the token
 * at position pos (the KV cache holds positions 0..pos-1); `steps` tokens to
 * out_tokens.  The steps replay the decoder's one-token step graph. */
int rai_greedy_decode(rai_lookup *dec, const uint32_t *context, size_t len, size_t pos, size_t steps,
                      uint32_t *out_tokens);
/* The `rai run` decode loop without speculation with a sampler (run.rs:692-735):
 * from a prefilled state as rai_greedy_decode, each token chosen by
 * apply_repetition_penalty over the whole context (sampler.rs:185-199) and
 * sample_token with the config (sampler.rs:47-182), drawing from the
 * decoder's StdRng (rai_lookup_seed).  Ties of equal probabilities in the
 * top-p order are taken lowest index first (the reference's unstable sort
 * leaves their order unspecified). */
int rai_sample_decode(rai_lookup *dec, const uint32_t *context, size_t len, size_t pos, size_t steps,
                      const rai_sampler_config *cfg, uint32_t *out_tokens);
/* apply_repetition_penalty over recent[0..n_recent) then sample_token with
 * the config (sampler.rs:47-199) on one host logit row, `draws` times in a
 * row (each on the unchanged row) from StdRng::seed_from_u64(seed): the
 * device sampler alone, for checks against another implementation. */
int rai_sample_tokens(const float *logits, size_t vocab, const uint32_t *recent, size_t n_recent,
                      const rai_sampler_config *cfg, uint64_t seed, size_t draws, uint32_t *out_tokens);

/* ------------------------------------------------------------------ misc -- */
/* Synthetic .raimodel writer (the build's stand-in for the exporter).
 * mode 0: symmetric int4 RTN (code = q+8, zero = -8*scale) of N(0, std)
 * weights from `seed`; mode 1: the reference exporter's asymmetric min/max RTN
 * (raimodel.py:257-303) over the same weights.  Norm vectors are 1.0.
 * Writes to `path`, or, when path is NULL, returns a malloc'ed image in
 * *image / *image_len (free with rai_free_image). */
typedef struct rai_synth_config {
  uint32_t hidden_size, num_layers, num_heads, num_kv_heads, head_dim;
  uint32_t intermediate_size, vocab_size, max_context;
  float rope_theta, norm_eps;
  uint32_t group_size, embed_group_size, tied;
  uint32_t num_experts, experts_per_token, norm_topk_prob;
  float weight_std;
  uint32_t mode;
} rai_synth_config;
int rai_synth_model(const rai_synth_config *cfg, uint64_t seed, const char *path, uint8_t **image,
                    size_t *image_len);
void rai_free_image(uint8_t *image);

/* Test hook (no reference counterpart): the poll limit of the attention
 * kernel's bounded tile hand-off waits for launches enqueued from now on
 * (<= 0 restores the default).  A tiny limit makes the waits give up; every
 * kernel still ends, and the call that ran it fails with RAI_E_HIP.  Step
 * graphs keep the limit they were captured with. */
int rai_debug_set_attention_spin(int polls);

/* Device-memory plumbing for harnesses that bind only this ABI. */
int rai_dev_malloc(size_t bytes, void **out);
int rai_dev_free(void *ptr);
int rai_memcpy_h2d(void *dst, const void *src, size_t bytes);
int rai_memcpy_d2h(void *dst, const void *src, size_t bytes);
int rai_device_synchronize(void);
/* Stream/event helpers for timing from a harness (HIP events). */
int rai_stream_create(void **out);
int rai_stream_destroy(void *stream);
int rai_event_create(void **out);
int rai_event_destroy(void *ev);
int rai_event_record(void *ev, void *stream);
int rai_event_elapsed_ms(void *start, void *stop, float *ms);
int rai_stream_synchronize(void *stream);

#ifdef __cplusplus
}
#endif
#endif /* RAI_HIP_H */
