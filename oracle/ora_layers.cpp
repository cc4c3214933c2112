// Oracle: transformer layer kernels, restated from rai-infer/src/layers.rs
// (AVX2 path).  Test infrastructure only; see oracle.h.
#include <immintrin.h>

#include <cmath>
#include <cstring>

#include "ora_internal.h"

namespace ora {

// rms_norm_avx2 (layers.rs:325-376): two 8-lane FMA accumulators over
// 16-element steps, one trailing 8-block into sq0, horizontal reduce, scalar
// tail; inv = 1/sqrt(sum/n + eps); out = (x*inv)*w.
static float sum_squares(const float *x, int n) {
  __m256 sq0 = _mm256_setzero_ps(), sq1 = _mm256_setzero_ps();
  int i = 0;
  const int c16 = (n / 8) / 2;
  for (int c = 0; c < c16; ++c) {
    __m256 v0 = _mm256_loadu_ps(x + i), v1 = _mm256_loadu_ps(x + i + 8);
    sq0 = _mm256_fmadd_ps(v0, v0, sq0);
    sq1 = _mm256_fmadd_ps(v1, v1, sq1);
    i += 16;
  }
  if (i + 8 <= n) {
    __m256 v0 = _mm256_loadu_ps(x + i);
    sq0 = _mm256_fmadd_ps(v0, v0, sq0);
    i += 8;
  }
  float s = hsum8(_mm256_add_ps(sq0, sq1));
  for (; i < n; ++i) s += x[i] * x[i];
  return s;
}

static void scale_by(float *out, const float *x, const float *w, int n, float inv) {
  const int c8 = n / 8;
  const __m256 inv_v = _mm256_set1_ps(inv);
  int i = 0;
  for (int c = 0; c < c8; ++c, i += 8)
    _mm256_storeu_ps(out + i, _mm256_mul_ps(_mm256_mul_ps(_mm256_loadu_ps(x + i), inv_v),
                                            _mm256_loadu_ps(w + i)));
  for (; i < n; ++i) out[i] = x[i] * inv * w[i];
}

void rms_norm(float *out, const float *x, const float *w, int n, float eps) {
  const float ss = sum_squares(x, n);
  const float inv = 1.0f / std::sqrt(ss / (float)n + eps);
  scale_by(out, x, w, n, inv);
}

// rms_norm_with_residual_avx2 (layers.rs:416-497): same arithmetic plus a copy.
void rms_norm_residual(float *normed, float *residual, const float *x, const float *w, int n,
                       float eps) {
  std::memcpy(residual, x, sizeof(float) * n);
  rms_norm(normed, x, w, n, eps);
}

// vec_add (layers.rs:503-531).
void vec_add(float *h, const float *r, const float *a, int n) {
  for (int i = 0; i < n; ++i) h[i] = r[i] + a[i];
}

// Schraudolph's exponential (N. Schraudolph, "A fast, compact approximation
// of the exponential function", Neural Computation 11(4), 1999), in the
// constants and operation order of layers.rs:855-876 / 1317-1331:
// bits = cvt_rne(clamp(12102203*x + (1065353216-486411), 0, 2139095040)).
static inline __m256 schraudolph8(__m256 x) {
  const __m256 a = _mm256_set1_ps(12102203.0f);
  const __m256 b = _mm256_set1_ps(1065353216.0f - 486411.0f);
  __m256 t = _mm256_add_ps(_mm256_mul_ps(a, x), b);
  t = _mm256_max_ps(_mm256_min_ps(t, _mm256_set1_ps(2139095040.0f)), _mm256_set1_ps(0.0f));
  return _mm256_castsi256_ps(_mm256_cvtps_epi32(t));
}

float schraudolph(float x) {
  float buf[8];
  _mm256_storeu_ps(buf, schraudolph8(_mm256_set1_ps(x)));
  return buf[0];
}

// silu_mul_avx2 (layers.rs:850-883): 8-wide Schraudolph body, exact-exp tail.
void silu_mul(float *gate, const float *up, int n) {
  const int c8 = n / 8;
  const __m256 one = _mm256_set1_ps(1.0f), neg_one = _mm256_set1_ps(-1.0f);
  for (int i = 0; i < c8; ++i) {
    __m256 x = _mm256_loadu_ps(gate + i * 8);
    __m256 u = _mm256_loadu_ps(up + i * 8);
    __m256 e = schraudolph8(_mm256_mul_ps(x, neg_one));
    __m256 s = _mm256_div_ps(x, _mm256_add_ps(one, e));
    _mm256_storeu_ps(gate + i * 8, _mm256_mul_ps(s, u));
  }
  for (int i = c8 * 8; i < n; ++i) {
    const float x = gate[i];
    gate[i] = x / (1.0f + std::exp(-x)) * up[i];
  }
}

// RoPETable::with_scaling, RopeScaling::None (layers.rs:561-633).
void rope_tables(std::vector<float> &cos_t, std::vector<float> &sin_t, int hd, int max_ctx,
                 float theta) {
  const int half = hd / 2;
  std::vector<float> inv(half);
  for (int i = 0; i < half; ++i) inv[i] = 1.0f / std::pow(theta, (2.0f * (float)i) / (float)hd);
  cos_t.assign((size_t)max_ctx * half, 0.0f);
  sin_t.assign((size_t)max_ctx * half, 0.0f);
  for (int p = 0; p < max_ctx; ++p)
    for (int i = 0; i < half; ++i) {
      const float ang = (float)p * inv[i];
      cos_t[(size_t)p * half + i] = std::cos(ang);
      sin_t[(size_t)p * half + i] = std::sin(ang);
    }
}

// RoPETable::apply_avx2 (layers.rs:689-726): half-split pairs (i, i+hd/2),
// fmsub/fmadd bodies, unfused scalar tail.
void rope_apply(float *heads, int num_heads, int hd, const float *c, const float *s) {
  const int half = hd / 2;
  const int c8 = half / 8;
  for (int h = 0; h < num_heads; ++h) {
    float *b = heads + h * hd;
    for (int k = 0; k < c8; ++k) {
      const int i = k * 8;
      __m256 cv = _mm256_loadu_ps(c + i), sv = _mm256_loadu_ps(s + i);
      __m256 x0 = _mm256_loadu_ps(b + i), x1 = _mm256_loadu_ps(b + half + i);
      __m256 r0 = _mm256_fmsub_ps(x0, cv, _mm256_mul_ps(x1, sv));
      __m256 r1 = _mm256_fmadd_ps(x1, cv, _mm256_mul_ps(x0, sv));
      _mm256_storeu_ps(b + i, r0);
      _mm256_storeu_ps(b + half + i, r1);
    }
    for (int i = c8 * 8; i < half; ++i) {
      const float x0 = b[i], x1 = b[half + i];
      b[i] = x0 * c[i] - x1 * s[i];
      b[half + i] = x1 * c[i] + x0 * s[i];
    }
  }
}

// attention_head_avx2 (layers.rs:1266-1380), softcap disabled.
void attention_head(const float *q, const float *k, const float *v, int pos, int hd, float scale,
                    float *out, float *scores) {
  const int c8 = hd / 8;
  float mx = -INFINITY;
  for (int t = 0; t <= pos; ++t) {
    const float *kt = k + (size_t)t * hd;
    __m256 acc = _mm256_setzero_ps();
    for (int c = 0; c < c8; ++c)
      acc = _mm256_fmadd_ps(_mm256_loadu_ps(q + c * 8), _mm256_loadu_ps(kt + c * 8), acc);
    const float sc = hsum8(acc) * scale;
    scores[t] = sc;
    if (sc > mx) mx = sc;
  }
  const int n = pos + 1;
  const int n8 = n / 8;
  const __m256 mv = _mm256_set1_ps(mx);
  __m256 sacc = _mm256_setzero_ps();
  for (int i = 0; i < n8; ++i) {
    __m256 e = schraudolph8(_mm256_sub_ps(_mm256_loadu_ps(scores + i * 8), mv));
    _mm256_storeu_ps(scores + i * 8, e);
    sacc = _mm256_add_ps(sacc, e);
  }
  float sum = hsum8(sacc);
  for (int t = n8 * 8; t < n; ++t) {
    const float e = std::exp(scores[t] - mx);
    scores[t] = e;
    sum += e;
  }
  const float inv = 1.0f / sum;
  const __m256 iv = _mm256_set1_ps(inv);
  for (int i = 0; i < n8; ++i)
    _mm256_storeu_ps(scores + i * 8, _mm256_mul_ps(_mm256_loadu_ps(scores + i * 8), iv));
  for (int t = n8 * 8; t < n; ++t) scores[t] *= inv;
  for (int c = 0; c < c8; ++c) _mm256_storeu_ps(out + c * 8, _mm256_setzero_ps());
  for (int t = 0; t <= pos; ++t) {
    const float *vt = v + (size_t)t * hd;
    const __m256 pv = _mm256_set1_ps(scores[t]);
    for (int c = 0; c < c8; ++c)
      _mm256_storeu_ps(out + c * 8,
                       _mm256_fmadd_ps(pv, _mm256_loadu_ps(vt + c * 8), _mm256_loadu_ps(out + c * 8)));
  }
}

// sampler.rs:201-208 argmax via f32::total_cmp, last maximum wins; the
// caller-side NaN -> -inf replacement of sample_token (sampler.rs:55-59) is
// folded in.
static inline int32_t total_key(float f) {
  int32_t b;
  std::memcpy(&b, &f, 4);
  return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

int64_t argmax(const float *v, int64_t n) {
  if (n <= 0) return 0;
  int64_t best = 0;
  int32_t bk = 0;
  for (int64_t i = 0; i < n; ++i) {
    float f = std::isnan(v[i]) ? -INFINITY : v[i];
    const int32_t k = total_key(f);
    if (i == 0 || k >= bk) {
      bk = k;
      best = i;
    }
  }
  return best;
}

}  // namespace ora
