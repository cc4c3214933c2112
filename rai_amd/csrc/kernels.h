// Launchers for the gfx950 kernels (kernels.hip).  All launchers are
// asynchronous on `stream` and validate nothing: callers check shapes.
#ifndef RAI_KERNELS_H
#define RAI_KERNELS_H

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace rai {

// Per-token activation quantization of gemm.rs:147-374 for K-column rows:
// q_nat [m][K] int8 in natural column order; q_split [m][K] int8 in
// 8-column blocks of (4 even columns, 4 odd columns) when K % 8 == 0 (else
// unused, may be null); scales/sums [m][groups].
void launch_quantize(const float *x, int m, int k, int gs, int8_t *q_nat, int8_t *q_split,
                     float *scales, float *sums, hipStream_t s);

// w4a8 matmul over already-quantized activations (see gemm.rs:1774-1919).
// `add` (may be null, may equal `out`): a residual [m][rows] added to each
// output, out = add + matmul (the reference's vec_add after o_proj/down,
// layers.rs:503-531, fused into the epilogue).
// `qa` (may be null): the activations packed by launch_qa_pack, which
// enables the matrix-core kernel for 2..kMfmaMaxTokens tokens at group 32.
// `mm` (may be null): mm_pack_bytes(m, cols) bytes of scratch, which
// enables the matrix-core GEMM for more than kMfmaMaxTokens tokens.
// `params_tiled` (may be null): launch_params_tile16's copy of `params`,
// which the matrix-core GEMV then reads.
void launch_w4a8(float *out, const float *add, const uint8_t *nib, const uint8_t *params, const float *x,
                 const int8_t *q_nat, const int8_t *q_split, const float *scales,
                 const float *sums, int rows, int cols, int m, int gs, hipStream_t s,
                 const _Float16 *qa = nullptr, uint8_t *mm = nullptr, const uint8_t *params_tiled = nullptr);

// One token: rms_norm(x) * norm_w (layers.rs:325-376), its group-32
// quantization and the W4A8 GEMV in one launch; each block normalises and
// quantizes the row into its own LDS (no workspace traffic).  Applies when
// w4a8_norm1_path holds (group 32, at most 128 groups); false otherwise.
bool w4a8_norm1_path(int rows, int cols, int gs);
bool launch_w4a8_norm1(float *out, const float *add, const uint8_t *nib, const uint8_t *params, const float *x,
                       const float *norm_w, float eps, int rows, int cols, int gs, hipStream_t s);

// One-token W4A8 GEMV, wave-streamed (decode_gemv.hip): group 32, K <= 14336.
// With nx/nw (K <= 4096) the kernel applies rms_norm(nx) * nw and the
// group-32 quantization itself (q_split, scales, sums unused); with nx alone
// it quantizes nx (quantize_input_split of the f32 row).  variant
// selects the tile height and ring depth, blocks the grid (0: one tile per
// wave).  False when the shape is not covered.
bool w4a8_dec_path(int rows, int cols, int gs);
bool launch_w4a8_dec(float *out, const float *add, const uint8_t *nib, const uint8_t *params, const int8_t *q_split,
                     const float *scales, const float *sums, int rows, int cols, int gs, const float *nx,
                     const float *nw, float eps, hipStream_t s, int variant = 0, int blocks = 0);

// One token through a stacked gate|up projection (rows = 2F, gate rows
// first): rms_norm(x) * norm_w, quantization, the GEMV, silu(gate) * up and
// the group-32 quantization of that product in one launch; writes only the
// quantized product (q_out [F] block-split, scale_out / sum_out [F / 32]).
// False when the shape is not covered (F % 32 != 0, K > 4096, ...).
bool launch_w4a8_glu1(const uint8_t *nib, const uint8_t *params, const float *x, const float *norm_w, float eps,
                      int rows, int cols, int gs, int8_t *q_out, float *scale_out, float *sum_out, hipStream_t s);

// Rotary embedding and KV store of one token, applied by a GEMV epilogue.
struct DecRope {
  const float *cos_t, *sin_t;  // [pos][hd / 2] tables
  int pos0;                    // token position (read from st[0] when st)
  const int *st;
  float *kc, *vc;              // K cache [nkv][cap][hd], V cache d-major [nkv][hd][vstride]
  int cap, vstride, nh, nkv, hd;
};
// One token through the stacked [q; k; v] projection (rows (nh + 2 nkv) hd):
// rms_norm(x) * norm_w, quantization, the GEMV, then rope_store's rotation of
// q and k, the K and V cache stores (as launch_rope_store for m = 1).
bool launch_w4a8_qkv_rope1(float *out, const uint8_t *nib, const uint8_t *params, const float *x,
                           const float *norm_w, float eps, int rows, int cols, int gs, const DecRope &rope,
                           hipStream_t s);

// Expert GEMVs (one-token kernel, one grid row per MoE entry): entry
// i = t * K + k is slot k of token t; with expert x = sel[i] in [0, E) it
// runs matrix (nib_tab[x * tstride], par_tab[x * tstride]) against
// activation row t (tok_rows) or i of q_split / scales / sums and writes
// out + i * ld; an empty slot (sel[i] < 0) leaves its row as it is.
struct DecMoe {
  const uint8_t *const *nib_tab, *const *par_tab;
  int tstride;
  const int *sel;
  int K;
  bool tok_rows;
  int E, ld;
  // Outputs of launch_w4a8_dec_moe_glu: per entry the quantized silu_mul
  // row (rows / 2 int8 in the block-split order), its scales and sums.
  int8_t *qo = nullptr;
  float *so = nullptr, *uo = nullptr;
};
bool launch_w4a8_dec_moe(float *out, const DecMoe &moe, const int8_t *q_split, const float *scales,
                         const float *sums, int rows, int cols, int gs, int max_entries, hipStream_t s);
// The experts' gate|up (rows = 2 F, gate rows first) with silu_mul_inplace
// and the quantization of its output fused (as launch_silu_quant): one block
// per (32-value output group, entry); false when the shape is outside the
// one-token kernel's (or rows % 64 != 0).
bool launch_w4a8_dec_moe_glu(const DecMoe &moe, const int8_t *q_split, const float *scales, const float *sums,
                             int rows, int cols, int gs, int max_entries, hipStream_t s);

// Matrix-core W4A8 (gemv.hip): group 32, K a multiple of 256, 2..64 tokens
// (past 64 the GEMM of gemm_mm.hip is faster on every measured shape).
constexpr int kMfmaMaxTokens = 64;
bool w4a8_mfma_path(int rows, int cols, int m, int gs);
// Halves of the packed activation buffer for m tokens of `cols` columns.
size_t qa_pack_halves(int m, int cols);
// Packs block-split int8 activations [m][cols] into the MFMA A-operand
// layout (f16, zero rows for the padding tokens of the last 4-token group).
void launch_qa_pack(const int8_t *q_split, int m, int cols, _Float16 *qa, hipStream_t s);
// `params_tiled` (may be null): the same parameters in the layout of
// launch_params_tile16, read instead of `params` where it applies.
// `q_split` (may be null): the block-split int8 activations the packed
// `qa` was made from, from which the register-pipelined kernel builds its
// A operands itself.
bool launch_w4a8_mfma(float *out, const float *add, const uint8_t *nib, const uint8_t *params, const _Float16 *qa,
                      const int8_t *q_split, const float *scales, const float *sums, int rows, int cols, int m,
                      int gs, hipStream_t s, const uint8_t *params_tiled = nullptr);
// The parameter array of a group-32 matrix (rows x cols/32 dwords, f16
// scale and zero point per row and group) rearranged in 16-row tiles:
// [rows / 16][cols / 128][16 rows][4 groups] dwords, the layout the
// matrix-core GEMV reads in one 256-byte piece per step and wave.  Same
// size as the input; requires params_tile16_ok.
bool params_tile16_ok(int rows, int cols, int gs);
void launch_params_tile16(const uint8_t *params, int rows, int cols, uint8_t *tiled, hipStream_t s);
// Matrix-core W4A8 GEMM (gemm_mm.hip): group 32, K a multiple of 512,
// more than kMfmaMaxTokens tokens.  Packs the block-split activations into
// `pack` (mm_pack_bytes(m, cols) bytes), then runs the GEMM.
bool w4a8_mm_path(int rows, int cols, int m, int gs);
size_t mm_pack_bytes(int m, int cols);
void launch_w4a8_mm(float *out, const float *add, const uint8_t *nib, const uint8_t *params, const int8_t *q_split,
                    const float *scales, const float *sums, int rows, int cols, int m, uint8_t *pack,
                    hipStream_t s);
// True when launch_w4a8 takes the tiled fast path for this shape.
bool w4a8_fast_path(int cols, int gs);

void launch_lane_sums(int32_t *out, const uint8_t *nib, const int8_t *q_nat, int rows, int cols,
                      int m, int gs, hipStream_t s);

// Tied 8-bit lm_head (gemm.rs:804-1047, 1981-2076) for m tokens.
void launch_tied_lm_head(float *logits, const float *hidden, const uint8_t *codes,
                         const uint8_t *params, int vocab, int n, int gs, int m, int8_t *hq,
                         float *hscales, float *hsums, hipStream_t s);

// Embedding rows (gemm.rs:1926-1970, model.rs:371-403) for token ids read
// from `tokens` (device), or, when tokens == null, from
// ctx[last] followed by ctx[start .. start+m-1) (the lookup verify batch).
// Device step record for graph replay: int[4] = {pos0, len, start, nd}.
// Kernels given one read their position arguments from it (the host
// arguments are then ignored); null means use the host arguments.
void launch_embed(const uint32_t *tokens, const uint32_t *ctx, int last, int start, int m,
                  const uint8_t *codes, const uint8_t *params, int vocab, int hidden, int egs,
                  float embed_scale, float *out, int *err, hipStream_t s,
                  const int *st = nullptr);

void launch_rmsnorm(const float *x, const float *w, float *out, float *resid, int m, int n,
                    float eps, hipStream_t s);

// Fused kernels (fused.hip).  fused_quant_ok: the row length and group size
// the fused quantizing kernels handle (group 32/64/128, whole groups).
bool fused_quant_ok(int n, int gs);
// RMSNorm of m rows of n (layers.rs:325-376) + per-group quantization of
// the result (gemm.rs:147-374); `normed` and `q_nat` may be null.
// qa (may be null; group 32 only): also write the quantized rows in the
// matrix-core activation layout (launch_qa_pack's output, padding rows of
// the last 4-token group left untouched), which saves that pack.
void launch_norm_quant(const float *x, const float *w, float *normed, int m, int n, float eps,
                       int gs, int8_t *q_split, int8_t *q_nat, float *scales, float *sums,
                       hipStream_t s, _Float16 *qa = nullptr);
// Per-group quantization of m rows of n into q_split (q_nat may be null).
void launch_quant(const float *x, int m, int n, int gs, int8_t *q_split, int8_t *q_nat,
                  float *scales, float *sums, hipStream_t s, _Float16 *qa = nullptr);
// silu_mul (layers.rs:850-883) in place on gate rows of n (row stride ld,
// up rows likewise) + quantization of the product; requires n % 8 == 0.
void launch_silu_quant(float *gate, const float *up, int m, int n, int ld, int gs,
                       int8_t *q_split, int8_t *q_nat, float *scales, float *sums,
                       hipStream_t s, _Float16 *qa = nullptr);
void launch_vec_add(float *h, const float *r, const float *a, size_t n, hipStream_t s);
void launch_silu_mul(float *gate, const float *up, int m, int n, hipStream_t s);
// RoPE on q [m][nh*hd] and k [m][nkv*hd] at positions pos0.., then the
// KV store: K into kc [nkv][cap][hd], V into vc d-major [nkv][hd][vstride].
// Rows of q are q_ld floats apart, rows of k and v kv_ld apart.
void launch_rope_store(float *q, float *k, const float *v, const float *cos_t, const float *sin_t,
                       int pos0, int m, int nh, int nkv, int hd, float *kc, float *vc, int cap,
                       int vstride, int q_ld, int kv_ld, hipStream_t s,
                       const int *st = nullptr);
// attention_head_avx2 for every (token, query head).  K cache [nkv][cap][hd];
// V cache d-major [nkv][hd][vstride] when vstride > 0, else [nkv][cap][hd].
// `scores` is scratch of attention_scores_floats(m, nh, pos0 + m) floats;
// tokens are processed in groups of kAttnTokens.
constexpr int kAttnTokens = 128;
size_t attention_scores_floats(int m, int nh, int ctx);
// q rows are q_ld floats apart; out is [m][nh * hd].
// With a step record `st` (m <= kAttnTokens), grids, the score stride and
// the softmax kernel are sized for a span of positions, min(cap, span), so
// the launch does not depend on the position (a captured step stays valid
// for every position below its span).  Spans are kAttnSpan0 << b:
// attn_span(cap, n) is the span of a step whose last position is n - 1, and
// attn_span_index its b.  `err` (may be null): bit 0 is set when a PV tile
// hand-off wait gave up (the output is then wrong and the caller must fail).
constexpr int kAttnSpan0 = 256;
inline int attn_span_index(int n) {
  int b = 0;
  while ((kAttnSpan0 << b) < n) ++b;
  return b;
}
inline int attn_span(int cap, int n) {
  const int s = kAttnSpan0 << attn_span_index(n);
  return s < cap ? s : cap;
}
// `stages` (timing only): bit 0 the score launch, bit 1 the softmax, bit 2
// PV; a stage left out uses what the buffers already hold.  `span`: see
// above (0 = the first span).
void launch_attention(const float *q, int q_ld, const float *kc, const float *vc, int cap,
                      int vstride, int pos0, int m, int nh, int nkv, int hd, float scale,
                      float *out, float *scores, hipStream_t s, const int *st = nullptr,
                      int *err = nullptr, int stages = 7, int span = 0);
// Poll limit of the PV tile hand-off waits for launches enqueued from now
// on (<= 0 restores the default).  Lowering it is for tests of the error
// path: the waits then give up and report it, and every block still ends.
void set_attention_spin(int polls);
// Standalone RoPE of one position (layers.rs:643-726) on heads [nh][hd].
void launch_rope_apply(float *heads, int nh, int hd, const float *cos_row, const float *sin_row,
                       hipStream_t s);
void launch_argmax(const float *logits, int m, int vocab, uint32_t *out, hipStream_t s);
// find_ngram_draft over ctx[0..len): res = {ngram, start, len}; ngram 0 = none.
void launch_ngram(const uint32_t *ctx, int len, int min_n, int max_n, int max_draft, int *res,
                  hipStream_t s);
// The next decoder step's search at the end of a step whose acceptance
// wrote {accepted, produced} to res_acc: over ctx[0..len + produced) for
// position pos + produced (draft capped by max_ctx).  With a step record
// `st`, pos, len and min_n / max_n / max_draft are read from st[0], st[1],
// st[5..7].
void launch_ngram_next(const uint32_t *ctx, int len, int pos, int min_n, int max_n, int max_draft, int max_ctx,
                       const int *res_acc, int *res, hipStream_t s, const int *st = nullptr);
// Greedy acceptance: argmax[0..nd] vs ctx[start..start+nd); writes the
// produced tokens to ctx[len..] and res2 = {accepted, produced}.
void launch_accept(const uint32_t *argmax, uint32_t *ctx, int len, int start, int nd, int *res2,
                   hipStream_t s, const int *st = nullptr);

// MoE (layers.rs:1808-1870, model.rs:208-261): router probabilities and
// top-k selection per token.
void launch_router(const float *x, const float *router, int m, int hidden, int experts, int topk,
                   int norm_topk, int *sel, float *wts, float *logits, hipStream_t s);
// out[t] += w * eo[t] for the m tokens (per-token weight array w[t]).
void launch_moe_accumulate(float *out, const float *eo, const float *w, int m, int n,
                           hipStream_t s);
void launch_fill(float *p, float v, size_t n, hipStream_t s);

// Exact-sampling acceptance (sample.hip).  The decoder's rand 0.8 StdRng
// (ChaCha12) in device memory: key, 64-bit block counter, the four-block
// word buffer and the read index (64 = empty).
struct RngState {
  uint32_t key[8];
  uint32_t counter_lo, counter_hi;
  int index, pad;
  uint32_t buf[64];
};
// SeedableRng::seed_from_u64 (host side).
void rng_seed_from_u64(RngState &r, uint64_t seed);
// k_sample_probs over `rows` verify rows (nd + 1), then the accept / correct
// / bonus loop; appends the produced tokens to ctx[len..] and writes
// res = {accepted, produced}.  With a step record st the kernels read len,
// start, nd (st[1..3]) and the temperature bits (st[4]) from it.  probs
// holds rows * V floats, scratch V floats.
void launch_sample(const float *logits, float *probs, int V, uint32_t *ctx, int len, int start, int nd, float T,
                   RngState *rng, float *scratch, int *res, hipStream_t s, const int *st, int rows);
// SpeculativeDecoder's phase 3 (speculative.rs:336-390): toks = [last,
// k drafts, outputs...]; target logits [k + 1][V], the drafts' logit rows
// [k][V]; appends the produced tokens at toks[k + 1..], res = {accepted,
// produced}.
void launch_spec_sample(const float *tlogits, float *tprobs, const float *dlogits, float *dprobs, int V,
                        uint32_t *toks, int k, float T, RngState *rng, float *scratch, int *res, hipStream_t s);
// One sampled draft token: keeps the row, draws *out with sample_token.
void launch_draw(const float *row, int V, float T, RngState *rng, float *keep, float *scratch, uint32_t *out,
                 hipStream_t s);
// n draws (kinds: 0 u32, 1 u64, 2 f32, 3 f64) from the device generator.
void launch_rng_draws(RngState *rng, const int *kinds, int n, uint64_t *out, hipStream_t s);
// apply_repetition_penalty over ctx[0..len), then sample_token with the whole
// SamplerConfig (sampler.rs:47-199) for one logit row: the token goes to
// tok_out (ctx[len] when null), res (may be null) = {0, 1}.  work: V floats;
// flags: V words, zero on entry and on exit.  With a step record, len, T
// and the options come from st[1], st[4], st[8..10].
void launch_sample_plain(const float *logits, int V, uint32_t *ctx, int len, float T, int top_k, float top_p,
                         float penalty, RngState *rng, float *work, uint32_t *flags, uint32_t *tok_out, int *res,
                         hipStream_t s, const int *st = nullptr);

// Device MoE (moe.hip): group 32/64/128, hidden and FFN multiples of 256,
// at most 1024 experts.
bool moe_device_path(int hidden, int ffn, int gs, int experts);
// ent_exp (may be null) receives each entry row's expert.
void launch_moe_plan(const int *sel, int m, int K, int E, int *off, int *ent_of, int *ent_tok, int *ent_exp,
                     hipStream_t s);
void launch_moe_gather(const int8_t *q, const float *sc, const float *su, const int *ent_tok, const int *off, int E,
                       int max_entries, int cols, int groups, int8_t *qg, float *scg, float *sug, hipStream_t s);
void launch_moe_gemv(float *out, int ld, const uint8_t *const *nibp, const uint8_t *const *parp, int nmat, int rows,
                     int cols, int gs, int E, const int8_t *q, const float *sc, const float *su, const int *off,
                     hipStream_t s);
void launch_moe_combine(float *hid, const float *eo, const float *wts, const int *ent_of, int m, int K, int H,
                        hipStream_t s);
// The combine with entries in (token, slot) order (entry t * K + k), empty
// slots marked by sel < 0.
void launch_moe_combine_sel(float *hid, const float *eo, const float *wts, const int *sel, int m, int K, int H,
                            hipStream_t s);

}  // namespace rai

#endif
