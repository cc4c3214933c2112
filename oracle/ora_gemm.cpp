// Oracle: W4A8 kernels, restated from rai-infer/src/gemm.rs (AVX2 path).
// Test infrastructure only; see oracle.h.
#include "ora_internal.h"

#include <immintrin.h>
#include <omp.h>

#include <cmath>
#include <cstring>

namespace ora {

// Horizontal sum of an 8-lane f32 accumulator in the reference's shuffle
// order: ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7))  (gemm.rs:193-199, 527-533).
float hsum8(__m256 acc) {
  __m128 hi = _mm256_extractf128_ps(acc, 1);
  __m128 lo = _mm256_castps256_ps128(acc);
  __m128 s = _mm_add_ps(lo, hi);
  __m128 sh = _mm_movehdup_ps(s);
  __m128 s2 = _mm_add_ps(s, sh);
  __m128 h2 = _mm_movehl_ps(s2, s2);
  return _mm_cvtss_f32(_mm_add_ss(s2, h2));
}

static inline float hmax8(__m256 v) {
  __m128 hi = _mm256_extractf128_ps(v, 1);
  __m128 lo = _mm256_castps256_ps128(v);
  __m128 m = _mm_max_ps(lo, hi);
  __m128 sh = _mm_movehdup_ps(m);
  __m128 m2 = _mm_max_ps(m, sh);
  __m128 h2 = _mm_movehl_ps(m2, m2);
  return _mm_cvtss_f32(_mm_max_ss(m2, h2));
}

float f16_to_f32(uint16_t h) {
  return _mm_cvtss_f32(_mm_cvtph_ps(_mm_cvtsi32_si128(h)));
}

// compute_input_sums_avx2 (gemm.rs:172-212).
void input_sums(const float *x, int cols, int gs, float *sums) {
  const int groups = (cols + gs - 1) / gs;
  for (int g = 0; g < groups; ++g) {
    const int start = g * gs;
    const int end = std::min((g + 1) * gs, cols);
    const int len = end - start;
    const int c8 = len / 8;
    __m256 acc = _mm256_setzero_ps();
    for (int i = 0; i < c8; ++i) acc = _mm256_add_ps(acc, _mm256_loadu_ps(x + start + i * 8));
    float total = hsum8(acc);
    for (int i = c8 * 8; i < len; ++i) total += x[start + i];
    sums[g] = total;
  }
}

// Rust's f32::round: half away from zero.
static inline float round_away(float v) { return std::round(v); }

// quantize_input_split_avx2 (gemm.rs:280-374).  Produces even/odd int8 columns
// and one scale per group.
void quantize_split(const float *x, int cols, int gs, int8_t *q_even, int8_t *q_odd,
                    float *scales) {
  const int groups = (cols + gs - 1) / gs;
  const __m256 sign_mask = _mm256_castsi256_ps(_mm256_set1_epi32(0x7FFFFFFF));
  const __m128i even_shuf = _mm_setr_epi8(0, 2, 4, 6, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1);
  const __m128i odd_shuf = _mm_setr_epi8(1, 3, 5, 7, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1);
  for (int g = 0; g < groups; ++g) {
    const int start = g * gs;
    const int end = std::min((g + 1) * gs, cols);
    const int len = end - start;
    const float *in = x + start;
    const int c8 = len / 8;
    __m256 vmax = _mm256_setzero_ps();
    for (int i = 0; i < c8; ++i)
      vmax = _mm256_max_ps(vmax, _mm256_and_ps(_mm256_loadu_ps(in + i * 8), sign_mask));
    float absmax = hmax8(vmax);
    for (int i = c8 * 8; i < len; ++i) {
      float a = std::fabs(in[i]);
      if (a > absmax) absmax = a;
    }
    const float scale = absmax > 1e-10f ? absmax / 127.0f : 1.0f;
    const float inv = 1.0f / scale;
    scales[g] = scale;
    const __m256 inv_v = _mm256_set1_ps(inv);
    const __m256 lo_v = _mm256_set1_ps(-128.0f);
    const __m256 hi_v = _mm256_set1_ps(127.0f);
    const int base = start / 2;
    for (int i = 0; i < c8; ++i) {
      __m256 v = _mm256_loadu_ps(in + i * 8);
      __m256 r = _mm256_round_ps(_mm256_mul_ps(v, inv_v), _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
      __m256 c = _mm256_max_ps(_mm256_min_ps(r, hi_v), lo_v);
      __m256i i32 = _mm256_cvtps_epi32(c);
      __m128i p16 = _mm_packs_epi32(_mm256_castsi256_si128(i32), _mm256_extracti128_si256(i32, 1));
      __m128i p8 = _mm_packs_epi16(p16, _mm_setzero_si128());
      int32_t e = _mm_cvtsi128_si32(_mm_shuffle_epi8(p8, even_shuf));
      int32_t o = _mm_cvtsi128_si32(_mm_shuffle_epi8(p8, odd_shuf));
      std::memcpy(q_even + base + i * 4, &e, 4);
      std::memcpy(q_odd + base + i * 4, &o, 4);
    }
    for (int col = start + c8 * 8; col + 1 < end; col += 2) {
      const int k = col / 2;
      q_even[k] = (int8_t)std::min(std::max(round_away(x[col] * inv), -128.0f), 127.0f);
      q_odd[k] = (int8_t)std::min(std::max(round_away(x[col + 1] * inv), -128.0f), 127.0f);
    }
  }
}

QuantInput quantize_token(const float *x, int cols, int gs) {
  QuantInput q;
  const int groups = (cols + gs - 1) / gs;
  q.even.assign(cols / 2, 0);
  q.odd.assign(cols / 2, 0);
  q.scales.assign(groups, 0.0f);
  q.sums.assign(groups, 0.0f);
  input_sums(x, cols, gs, q.sums.data());
  quantize_split(x, cols, gs, q.even.data(), q.odd.data(), q.scales.data());
  q.x = x;
  return q;
}

// Decode the f16 (scale, zero) of one row into two arrays (F16C, gemm.rs:444-452).
static void decode_row_params(const uint8_t *params, int row, int groups, float *ws, float *wz) {
  const uint8_t *p = params + (size_t)row * groups * 4;
  for (int g = 0; g < groups; ++g) {
    uint32_t bits;
    std::memcpy(&bits, p + g * 4, 4);
    __m128 f = _mm_cvtph_ps(_mm_cvtsi32_si128((int)bits));
    ws[g] = _mm_cvtss_f32(f);
    wz[g] = _mm_cvtss_f32(_mm_shuffle_ps(f, f, 1));
  }
}

// One weight row against one quantized token: the exact lane/group order of
// matvec_chunk_i8 (gemm.rs:401-539) and matmul_row_tile (gemm.rs:562-674),
// which are bit-identical to each other.
float row_dot(const uint8_t *nib_row, const float *ws, const float *wz, const QuantInput &q,
              int cols, int gs) {
  const int groups = (cols + gs - 1) / gs;
  const __m256i mask_0f = _mm256_set1_epi8(0x0F);
  const __m256i ones16 = _mm256_set1_epi16(1);
  __m256 facc = _mm256_setzero_ps();
  for (int g = 0; g < groups; ++g) {
    const int col0 = g * gs;
    const int ags = std::min((g + 1) * gs, cols) - col0;
    const int off = col0 / 2;
    const int c64 = ags / 64;
    __m256i iacc = _mm256_setzero_si256();
    for (int c = 0; c < c64; ++c) {
      __m256i raw = _mm256_loadu_si256((const __m256i *)(nib_row + off + c * 32));
      __m256i lo = _mm256_and_si256(raw, mask_0f);
      __m256i hi = _mm256_and_si256(_mm256_srli_epi16(raw, 4), mask_0f);
      __m256i ie = _mm256_loadu_si256((const __m256i *)(q.even.data() + off + c * 32));
      __m256i io = _mm256_loadu_si256((const __m256i *)(q.odd.data() + off + c * 32));
      __m256i comb = _mm256_add_epi16(_mm256_maddubs_epi16(lo, ie), _mm256_maddubs_epi16(hi, io));
      iacc = _mm256_add_epi32(iacc, _mm256_madd_epi16(comb, ones16));
    }
    const float cs = ws[g] * q.scales[g];
    facc = _mm256_add_ps(facc, _mm256_mul_ps(_mm256_cvtepi32_ps(iacc), _mm256_set1_ps(cs)));
    const int done = c64 * 64;
    const bool has32 = done + 32 <= ags;
    if (has32) {
      __m128i raw = _mm_loadu_si128((const __m128i *)(nib_row + off + done / 2));
      __m128i lo = _mm_and_si128(raw, _mm_set1_epi8(0x0F));
      __m128i hi = _mm_and_si128(_mm_srli_epi16(raw, 4), _mm_set1_epi8(0x0F));
      __m128i ie = _mm_loadu_si128((const __m128i *)(q.even.data() + off + done / 2));
      __m128i io = _mm_loadu_si128((const __m128i *)(q.odd.data() + off + done / 2));
      __m128i comb = _mm_add_epi16(_mm_maddubs_epi16(lo, ie), _mm_maddubs_epi16(hi, io));
      __m128i sums = _mm_madd_epi16(comb, _mm_set1_epi16(1));
      __m128 tail = _mm_mul_ps(_mm_cvtepi32_ps(sums), _mm_set1_ps(cs));
      facc = _mm256_add_ps(facc, _mm256_insertf128_ps(_mm256_setzero_ps(), tail, 0));
    }
    const int done2 = done + (has32 ? 32 : 0);
    if (done2 < ags) {
      // Unquantized f32 tail, lane 0 (gemm.rs:503-515).
      float tacc = 0.0f;
      for (int tc = done2; tc + 1 < ags; tc += 2) {
        const uint8_t b = nib_row[off + tc / 2];
        float a0 = (float)(b & 0x0F) * q.x[col0 + tc];
        float a1 = (float)(b >> 4) * q.x[col0 + tc + 1];
        tacc += a0 + a1;
      }
      facc = _mm256_add_ps(facc, _mm256_set_ps(0, 0, 0, 0, 0, 0, 0, ws[g] * tacc));
    }
  }
  const float dot = hsum8(facc);
  float zc = 0.0f;
  for (int g = 0; g < groups; ++g) zc += wz[g] * q.sums[g];
  return dot + zc;
}

void lane_sums(const uint8_t *nib_row, const QuantInput &q, int cols, int gs, int32_t *out) {
  const int groups = (cols + gs - 1) / gs;
  const __m256i mask_0f = _mm256_set1_epi8(0x0F);
  const __m256i ones16 = _mm256_set1_epi16(1);
  for (int g = 0; g < groups; ++g) {
    int32_t *o = out + g * 12;
    std::memset(o, 0, 12 * sizeof(int32_t));
    const int col0 = g * gs;
    const int ags = std::min((g + 1) * gs, cols) - col0;
    const int off = col0 / 2;
    const int c64 = ags / 64;
    __m256i iacc = _mm256_setzero_si256();
    for (int c = 0; c < c64; ++c) {
      __m256i raw = _mm256_loadu_si256((const __m256i *)(nib_row + off + c * 32));
      __m256i lo = _mm256_and_si256(raw, mask_0f);
      __m256i hi = _mm256_and_si256(_mm256_srli_epi16(raw, 4), mask_0f);
      __m256i ie = _mm256_loadu_si256((const __m256i *)(q.even.data() + off + c * 32));
      __m256i io = _mm256_loadu_si256((const __m256i *)(q.odd.data() + off + c * 32));
      __m256i comb = _mm256_add_epi16(_mm256_maddubs_epi16(lo, ie), _mm256_maddubs_epi16(hi, io));
      iacc = _mm256_add_epi32(iacc, _mm256_madd_epi16(comb, ones16));
    }
    _mm256_storeu_si256((__m256i *)o, iacc);
    const int done = c64 * 64;
    if (done + 32 <= ags) {
      __m128i raw = _mm_loadu_si128((const __m128i *)(nib_row + off + done / 2));
      __m128i lo = _mm_and_si128(raw, _mm_set1_epi8(0x0F));
      __m128i hi = _mm_and_si128(_mm_srli_epi16(raw, 4), _mm_set1_epi8(0x0F));
      __m128i ie = _mm_loadu_si128((const __m128i *)(q.even.data() + off + done / 2));
      __m128i io = _mm_loadu_si128((const __m128i *)(q.odd.data() + off + done / 2));
      __m128i comb = _mm_add_epi16(_mm_maddubs_epi16(lo, ie), _mm_maddubs_epi16(hi, io));
      _mm_storeu_si128((__m128i *)(o + 8), _mm_madd_epi16(comb, _mm_set1_epi16(1)));
    }
  }
}

// w4a8_matmul (gemm.rs:1774-1919); M = 1 is w4a8_matvec (gemm.rs:1336-1384).
// Rows are independent, so the OpenMP split does not change any result.
void matmul(float *out, const uint8_t *nib, const uint8_t *params, const float *x, int rows,
            int cols, int m, int gs) {
  const int groups = (cols + gs - 1) / gs;
  std::vector<QuantInput> qs;
  qs.reserve(m);
  for (int t = 0; t < m; ++t) qs.push_back(quantize_token(x + (size_t)t * cols, cols, gs));
  const size_t row_bytes = (size_t)cols / 2;
#pragma omp parallel
  {
    std::vector<float> ws(groups), wz(groups);
#pragma omp for schedule(static)
    for (int r = 0; r < rows; ++r) {
      decode_row_params(params, r, groups, ws.data(), wz.data());
      for (int t = 0; t < m; ++t)
        out[(size_t)t * rows + r] = row_dot(nib + r * row_bytes, ws.data(), wz.data(), qs[t], cols, gs);
    }
  }
}

// quantize_hidden_i8_avx2 (gemm.rs:924-1047): symmetric +-63 per group.
static void quantize_hidden_i8(const float *h, int n, int gs, int8_t *out, float *scales) {
  const int groups = (n + gs - 1) / gs;
  const __m256 sign_mask = _mm256_castsi256_ps(_mm256_set1_epi32(0x7FFFFFFF));
  for (int g = 0; g < groups; ++g) {
    const int start = g * gs;
    const int end = std::min((g + 1) * gs, n);
    const int len = end - start;
    const float *in = h + start;
    const int c8 = len / 8;
    __m256 vmax = _mm256_setzero_ps();
    for (int i = 0; i < c8; ++i)
      vmax = _mm256_max_ps(vmax, _mm256_and_ps(_mm256_loadu_ps(in + i * 8), sign_mask));
    float absmax = hmax8(vmax);
    for (int i = c8 * 8; i < len; ++i) {
      float a = std::fabs(in[i]);
      if (a > absmax) absmax = a;
    }
    const float scale = absmax > 1e-10f ? absmax / 63.0f : 1.0f;
    const float inv = 1.0f / scale;
    scales[g] = scale;
    const __m256 inv_v = _mm256_set1_ps(inv);
    for (int i = 0; i < c8; ++i) {
      __m256 v = _mm256_loadu_ps(in + i * 8);
      __m256 r = _mm256_round_ps(_mm256_mul_ps(v, inv_v), _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
      __m256 c = _mm256_max_ps(_mm256_min_ps(r, _mm256_set1_ps(63.0f)), _mm256_set1_ps(-63.0f));
      __m256i i32 = _mm256_cvtps_epi32(c);
      __m128i p16 = _mm_packs_epi32(_mm256_castsi256_si128(i32), _mm256_extracti128_si256(i32, 1));
      __m128i p8 = _mm_packs_epi16(p16, _mm_setzero_si128());
      int64_t bytes = _mm_cvtsi128_si64(p8);
      std::memcpy(out + start + i * 8, &bytes, 8);
    }
    for (int i = c8 * 8; i < len; ++i)
      out[start + i] = (int8_t)std::min(std::max(round_away(in[i] * inv), -63.0f), 63.0f);
  }
}

// tied_lm_head + lm_head_chunk_i8 (gemm.rs:804-915, 1981-2076).
void tied_lm_head(float *logits, const float *hidden, const uint8_t *codes,
                  const uint8_t *params, int vocab, int n, int gs) {
  const int groups = (n + gs - 1) / gs;
  std::vector<float> hsums(groups), hscales(groups);
  std::vector<int8_t> hq(n);
  input_sums(hidden, n, gs, hsums.data());
  quantize_hidden_i8(hidden, n, gs, hq.data(), hscales.data());
#pragma omp parallel
  {
    std::vector<float> ws(groups), wz(groups);
    const __m256i ones16 = _mm256_set1_epi16(1);
#pragma omp for schedule(static)
    for (int v = 0; v < vocab; ++v) {
      const uint8_t *row = codes + (size_t)v * n;
      decode_row_params(params, v, groups, ws.data(), wz.data());
      float zc = 0.0f;
      for (int g = 0; g < groups; ++g) zc += wz[g] * hsums[g];
      __m256 facc = _mm256_setzero_ps();
      for (int g = 0; g < groups; ++g) {
        const int col0 = g * gs;
        const int ags = std::min((g + 1) * gs, n) - col0;
        const int c32 = ags / 32;
        __m256i iacc = _mm256_setzero_si256();
        for (int c = 0; c < c32; ++c) {
          __m256i cv = _mm256_loadu_si256((const __m256i *)(row + col0 + c * 32));
          __m256i hv = _mm256_loadu_si256((const __m256i *)(hq.data() + col0 + c * 32));
          iacc = _mm256_add_epi32(iacc, _mm256_madd_epi16(_mm256_maddubs_epi16(cv, hv), ones16));
        }
        const float cs = ws[g] * hscales[g];
        facc = _mm256_add_ps(facc, _mm256_mul_ps(_mm256_cvtepi32_ps(iacc), _mm256_set1_ps(cs)));
        if (c32 * 32 < ags) {
          float tail = 0.0f;
          for (int i = c32 * 32; i < ags; ++i) tail += (float)row[col0 + i] * (float)hq[col0 + i];
          facc = _mm256_add_ps(facc, _mm256_set_ps(0, 0, 0, 0, 0, 0, 0, ws[g] * hscales[g] * tail));
        }
      }
      logits[v] = hsum8(facc) + zc;
    }
  }
}

// embed_lookup (gemm.rs:1926-1970): code*scale + zero, unfused.
void embed_lookup(float *out, int token, const uint8_t *codes, const uint8_t *params, int n,
                  int gs) {
  const int groups = (n + gs - 1) / gs;
  const uint8_t *row = codes + (size_t)token * n;
  const uint8_t *p = params + (size_t)token * groups * 4;
  for (int g = 0; g < groups; ++g) {
    uint16_t sb, zb;
    std::memcpy(&sb, p + g * 4, 2);
    std::memcpy(&zb, p + g * 4 + 2, 2);
    const float s = f16_to_f32(sb), z = f16_to_f32(zb);
    const int end = std::min((g + 1) * gs, n);
    for (int c = g * gs; c < end; ++c) out[c] = (float)row[c] * s + z;
  }
}

}  // namespace ora
