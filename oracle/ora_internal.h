// Oracle internals (test infrastructure only; see oracle.h).
#ifndef RAI_ORA_INTERNAL_H
#define RAI_ORA_INTERNAL_H

#include <immintrin.h>

#include <algorithm>
#include <cstdint>
#include <string>
#include <vector>

namespace ora {

// One token's activations quantized the reference way (gemm.rs:218-374):
// per-group int8 split into even/odd columns, per-group scales, and the
// per-group f32 sums of the raw input.
struct QuantInput {
  std::vector<int8_t> even, odd;
  std::vector<float> scales, sums;
  const float *x = nullptr;  // raw f32 input (the unquantized tail reads it)
};

float hsum8(__m256 acc);
float f16_to_f32(uint16_t h);
void input_sums(const float *x, int cols, int gs, float *sums);
void quantize_split(const float *x, int cols, int gs, int8_t *q_even, int8_t *q_odd,
                    float *scales);
QuantInput quantize_token(const float *x, int cols, int gs);
float row_dot(const uint8_t *nib_row, const float *ws, const float *wz, const QuantInput &q,
              int cols, int gs);
void lane_sums(const uint8_t *nib_row, const QuantInput &q, int cols, int gs, int32_t *out);
void matmul(float *out, const uint8_t *nib, const uint8_t *params, const float *x, int rows,
            int cols, int m, int gs);
void tied_lm_head(float *logits, const float *hidden, const uint8_t *codes,
                  const uint8_t *params, int vocab, int n, int gs);
void embed_lookup(float *out, int token, const uint8_t *codes, const uint8_t *params, int n,
                  int gs);

void rms_norm(float *out, const float *x, const float *w, int n, float eps);
void rms_norm_residual(float *normed, float *residual, const float *x, const float *w, int n,
                       float eps);
void vec_add(float *h, const float *r, const float *a, int n);
void silu_mul(float *gate, const float *up, int n);
void rope_tables(std::vector<float> &cos_t, std::vector<float> &sin_t, int hd, int max_ctx,
                 float theta);
void rope_apply(float *heads, int num_heads, int hd, const float *cos_row, const float *sin_row);
// k/v rows at stride hd, positions 0..=pos
void attention_head(const float *q, const float *k, const float *v, int pos, int hd, float scale,
                    float *out, float *scores);
float schraudolph(float x);

int64_t argmax(const float *v, int64_t n);

void set_error(const std::string &msg);

}  // namespace ora

// C-ABI body: run the statements, map an exception to -1 and the message.
#define ORA_TRY(...)                    \
  try {                                 \
    __VA_ARGS__;                        \
    return 0;                           \
  } catch (const std::exception &e) {   \
    ora::set_error(e.what());           \
    return -1;                          \
  }

#endif
