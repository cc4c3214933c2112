// CPU oracle: exact-sampling prompt-lookup (TEST INFRASTRUCTURE ONLY).
//
// Restates, for the checker:
//   - rand 0.8.6 StdRng = rand_chacha 0.3.1 ChaCha12Rng over rand_core 0.6.4
//     BlockRng (Cargo.lock of the reference): the ChaCha block function
//     (RFC 8439 quarter rounds; 64-bit block counter in words 12-13, 64-bit
//     stream in words 14-15, both zero-based), four blocks per refill, words
//     consumed in order; next_u64 = low word then high word, straddling a
//     refill as BlockRng does; SeedableRng::seed_from_u64 (PCG32 output
//     function filling the 32-byte key); Standard f32 = (u32 >> 8) * 2^-24,
//     f64 = (u64 >> 11) * 2^-53.
//   - softmax_probabilities and sample_correction (speculative.rs:414-513),
//     sample_token with top_k = 0, top_p = 1 (sampler.rs:47-182), and the
//     accept / correct / bonus loop of LookupDecoder::step (lookup.rs:359-403);
//   - apply_repetition_penalty and sample_token with the whole SamplerConfig
//     (sampler.rs:47-199), the token of `rai run` without speculation.
// Pins: the block function and the buffering order are checked against the
// RFC 7539 A.1 keystream vectors (20 rounds) and the RFC 8439 2.3.2 block;
// seed_from_u64 against the PCG32 reference demo's outputs (seed 42,
// sequence 54) through seeds that put its first step on the demo's states;
// the float conversions against rand 0.8's value-stability vectors.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <utility>
#include <vector>

#include "ora_internal.h"
#include "oracle.h"

namespace ora {

// f32::total_cmp order as an unsigned key (larger key = larger value).
static inline uint32_t total_key(float x) {
  uint32_t b;
  std::memcpy(&b, &x, 4);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

static inline uint32_t rotl(uint32_t x, int r) { return (x << r) | (x >> (32 - r)); }

static inline void quarter(uint32_t *s, int a, int b, int c, int d) {
  s[a] += s[b]; s[d] = rotl(s[d] ^ s[a], 16);
  s[c] += s[d]; s[b] = rotl(s[b] ^ s[c], 12);
  s[a] += s[b]; s[d] = rotl(s[d] ^ s[a], 8);
  s[c] += s[d]; s[b] = rotl(s[b] ^ s[c], 7);
}

void chacha_block(const uint32_t key[8], uint64_t counter, uint64_t stream, int rounds, uint32_t out[16]) {
  uint32_t in[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u};
  for (int i = 0; i < 8; ++i) in[4 + i] = key[i];
  in[12] = (uint32_t)counter;
  in[13] = (uint32_t)(counter >> 32);
  in[14] = (uint32_t)stream;
  in[15] = (uint32_t)(stream >> 32);
  uint32_t s[16];
  std::memcpy(s, in, sizeof(s));
  for (int r = 0; r < rounds; r += 2) {
    quarter(s, 0, 4, 8, 12);
    quarter(s, 1, 5, 9, 13);
    quarter(s, 2, 6, 10, 14);
    quarter(s, 3, 7, 11, 15);
    quarter(s, 0, 5, 10, 15);
    quarter(s, 1, 6, 11, 12);
    quarter(s, 2, 7, 8, 13);
    quarter(s, 3, 4, 9, 14);
  }
  for (int i = 0; i < 16; ++i) out[i] = s[i] + in[i];
}

// rand 0.8.6 Standard for f32 / f64 (distributions/float.rs): the top 24 /
// 53 bits of a u32 / u64 times 2^-24 / 2^-53.
static float standard_f32(uint32_t u) { return (float)(u >> 8) * (1.0f / 16777216.0f); }
static double standard_f64(uint64_t u) { return (double)(u >> 11) * (1.0 / 9007199254740992.0); }

struct StdRng {
  uint32_t key[8];
  uint64_t counter = 0;
  int rounds = 12;
  uint32_t buf[64];
  int index = 64;
  void refill() {
    for (int b = 0; b < 4; ++b) chacha_block(key, counter + b, 0, rounds, buf + 16 * b);
    counter += 4;
  }
  uint32_t next_u32() {
    if (index >= 64) {
      refill();
      index = 0;
    }
    return buf[index++];
  }
  uint64_t next_u64() {
    if (index < 63) {
      const uint64_t v = (uint64_t)buf[index] | ((uint64_t)buf[index + 1] << 32);
      index += 2;
      return v;
    }
    if (index >= 64) {
      refill();
      index = 2;
      return (uint64_t)buf[0] | ((uint64_t)buf[1] << 32);
    }
    const uint64_t lo = buf[63];
    refill();
    index = 1;
    return lo | ((uint64_t)buf[0] << 32);
  }
  float gen_f32() { return standard_f32(next_u32()); }
  double gen_f64() { return standard_f64(next_u64()); }
};

static void seed_from_u64(StdRng &r, uint64_t state) {
  const uint64_t mul = 6364136223846793005ull, inc = 11634580027462260723ull;
  for (int i = 0; i < 8; ++i) {
    state = state * mul + inc;
    const uint32_t xs = (uint32_t)(((state >> 18) ^ state) >> 27);
    const uint32_t rot = (uint32_t)(state >> 59);
    r.key[i] = (xs >> rot) | (xs << ((32 - rot) & 31));
  }
  r.counter = 0;
  r.index = 64;
}

// speculative.rs:431-477.
static std::vector<float> softmax_probabilities(const float *logits, int n, float temperature) {
  const float temp = (std::isfinite(temperature) && temperature > 1e-6f) ? temperature : 1.0f;
  std::vector<float> v(n);
  for (int i = 0; i < n; ++i) {
    const float x = logits[i] / temp;
    v[i] = std::isnan(x) ? -INFINITY : x;
  }
  int pinf = 0;
  for (int i = 0; i < n; ++i) pinf += v[i] == INFINITY;
  if (pinf > 0) {
    const float p = 1.0f / (float)pinf;
    for (int i = 0; i < n; ++i) v[i] = v[i] == INFINITY ? p : 0.0f;
    return v;
  }
  float mx = -INFINITY;
  for (int i = 0; i < n; ++i) mx = std::fmax(mx, v[i]);
  if (mx == -INFINITY) return std::vector<float>(n, 1.0f / (float)n);
  float sum = 0.0f;
  for (int i = 0; i < n; ++i) {
    v[i] = std::exp(v[i] - mx);
    sum += v[i];
  }
  if (!std::isfinite(sum) || sum <= 0.0f) return std::vector<float>(n, 1.0f / (float)n);
  for (int i = 0; i < n; ++i) v[i] /= sum;
  return v;
}

// sample_token (sampler.rs:47-182) with top_k = 0 and top_p = 1.
static int sample_token(std::vector<float> v, float temperature, StdRng &rng) {
  const int n = (int)v.size();
  if (n == 0) return 0;
  for (float &x : v)
    if (std::isnan(x)) x = -INFINITY;
  if (!std::isfinite(temperature) || temperature <= 1e-6f) return (int)argmax(v.data(), n);
  const float inv_temp = 1.0f / temperature;
  for (float &x : v) x *= inv_temp;
  int pinf = 0;
  for (float x : v) pinf += x == INFINITY;
  if (pinf > 0) {
    const float p = 1.0f / (float)pinf;
    for (float &x : v) x = x == INFINITY ? p : 0.0f;
  } else {
    float mx = -INFINITY;
    for (float x : v) mx = std::fmax(mx, x);
    if (mx == -INFINITY) {
      for (float &x : v) x = 1.0f / (float)n;
    } else {
      float sum = 0.0f;
      for (float &x : v) {
        x = std::exp(x - mx);
        sum += x;
      }
      if (std::isfinite(sum) && sum > 0.0f) {
        const float inv = 1.0f / sum;
        for (float &x : v) x *= inv;
      } else {
        for (float &x : v) x = 1.0f / (float)n;
      }
    }
  }
  const float r = rng.gen_f32();
  float cum = 0.0f;
  for (int i = 0; i < n; ++i) {
    cum += v[i];
    if (r < cum) return i;
  }
  return (int)argmax(v.data(), n);
}

// SamplerConfig (sampler.rs:17-42).
struct SamplerCfg {
  float temperature;
  int64_t top_k;
  float top_p;
};

// apply_repetition_penalty (sampler.rs:185-199): each distinct token of
// `recent` inside the vocabulary once: a positive logit divided by the
// penalty, any other multiplied; a non-finite, non-positive or ~1 penalty
// changes nothing.
static void apply_repetition_penalty(float *logits, int n, const int32_t *recent, int nr, float penalty) {
  if (!std::isfinite(penalty) || penalty <= 0.0f || std::fabs(penalty - 1.0f) < 1e-6f) return;
  std::vector<char> seen(n, 0);
  for (int i = 0; i < nr; ++i) {
    const int t = recent[i];
    if (t < 0 || t >= n || seen[t]) continue;
    seen[t] = 1;
    if (logits[t] > 0.0f)
      logits[t] /= penalty;
    else
      logits[t] *= penalty;
  }
}

// sample_token (sampler.rs:47-182) with the whole SamplerConfig, in its
// order: NaN -> -inf; greedy at T <= 1e-6 (or non-finite T); x * (1/T);
// top-k keeps x >= the k-th largest value (f32::total_cmp order for the
// selection, the plain comparison for the filter); the softmax (+inf
// entries share the mass, all -inf is uniform, exp and an f32 sum in index
// order, multiply by 1/sum, a degenerate sum is uniform); top-p (clamped to
// [0, 1], NaN = 1) keeps the candidates p > 1e-10 sorted by p descending up
// to the first cumulative f32 sum >= top_p, zeroes the rest and divides by
// the f32 sum in index order; then the cumulative search of one f32 draw,
// argmax as the fallback.  Ties of equal probabilities in the top-p order
// are taken lowest index first (the reference sorts with sort_unstable_by,
// which leaves their order unspecified).
static int sample_token_cfg(std::vector<float> v, const SamplerCfg &cfg, StdRng &rng) {
  const int n = (int)v.size();
  if (n == 0) return 0;
  for (float &x : v)
    if (std::isnan(x)) x = -INFINITY;
  if (!std::isfinite(cfg.temperature) || cfg.temperature <= 1e-6f) return (int)argmax(v.data(), n);
  const float inv_temp = 1.0f / cfg.temperature;
  for (float &x : v) x *= inv_temp;
  if (cfg.top_k > 0 && cfg.top_k < n) {
    std::vector<float> vals(v);
    const size_t k = (size_t)cfg.top_k;
    std::nth_element(vals.begin(), vals.begin() + (k - 1), vals.end(), [](float a, float b) {
      return total_key(a) > total_key(b);
    });
    const float threshold = vals[k - 1];
    for (float &x : v)
      if (x < threshold) x = -INFINITY;
  }
  int pinf = 0;
  for (float x : v) pinf += x == INFINITY;
  if (pinf > 0) {
    const float p = 1.0f / (float)pinf;
    for (float &x : v) x = x == INFINITY ? p : 0.0f;
  } else {
    float mx = -INFINITY;
    for (float x : v) mx = std::fmax(mx, x);
    if (mx == -INFINITY) {
      for (float &x : v) x = 1.0f / (float)n;
    } else {
      float sum = 0.0f;
      for (float &x : v) {
        x = std::exp(x - mx);
        sum += x;
      }
      if (std::isfinite(sum) && sum > 0.0f) {
        const float inv = 1.0f / sum;
        for (float &x : v) x *= inv;
      } else {
        for (float &x : v) x = 1.0f / (float)n;
      }
    }
  }
  const float top_p = std::isfinite(cfg.top_p) ? std::fmin(std::fmax(cfg.top_p, 0.0f), 1.0f) : 1.0f;
  if (top_p < 1.0f) {
    std::vector<std::pair<int, float>> cand;
    for (int i = 0; i < n; ++i)
      if (v[i] > 1e-10f) cand.emplace_back(i, v[i]);
    std::stable_sort(cand.begin(), cand.end(), [](const std::pair<int, float> &a, const std::pair<int, float> &b) {
      return total_key(a.second) > total_key(b.second);
    });
    float cum = 0.0f;
    size_t cutoff = cand.size();
    for (size_t r = 0; r < cand.size(); ++r) {
      cum += cand[r].second;
      if (cum >= top_p) {
        cutoff = r + 1;
        break;
      }
    }
    for (float &x : v) x = 0.0f;
    for (size_t r = 0; r < cutoff; ++r) v[cand[r].first] = cand[r].second;
    float sum = 0.0f;
    for (float x : v) sum += x;
    if (sum > 0.0f) {
      const float inv = 1.0f / sum;
      for (float &x : v) x *= inv;
    }
  }
  const float r = rng.gen_f32();
  float cum = 0.0f;
  for (int i = 0; i < n; ++i) {
    cum += v[i];
    if (r < cum) return i;
  }
  return (int)argmax(v.data(), n);
}

// The `rai run` plain decode token (run.rs:720-721): the penalty over the
// whole context, then sample_token.
int sample_plain(const float *logits, int n, const int32_t *ctx, int len, float temperature, int64_t top_k,
                 float top_p, float penalty, StdRng &rng) {
  std::vector<float> v(logits, logits + n);
  apply_repetition_penalty(v.data(), n, ctx, len, penalty);
  return sample_token_cfg(std::move(v), SamplerCfg{temperature, top_k, top_p}, rng);
}

// sample_correction (speculative.rs:479-513) against a point-mass draft on
// `draft` (all other draft logits -inf).
static int sample_correction(const float *target, int n, int draft, float temperature, StdRng &rng) {
  const std::vector<float> tp = softmax_probabilities(target, n, temperature);
  double adj_sum = 0.0;
  std::vector<float> adj(n);
  for (int i = 0; i < n; ++i) {
    const float dp = i == draft ? 1.0f : 0.0f;
    adj[i] = std::fmax(tp[i] - dp, 0.0f);
    adj_sum += (double)adj[i];
  }
  if (!std::isfinite(adj_sum) || adj_sum <= 0.0)
    return sample_token(std::vector<float>(target, target + n), temperature, rng);
  const double u = rng.gen_f64() * adj_sum;
  double cum = 0.0;
  for (int i = 0; i < n; ++i) {
    cum += (double)adj[i];
    if (cum >= u) return i;
  }
  return n - 1;
}

// The accept / correct / bonus loop of lookup.rs:359-403 over verify logits
// [nd + 1][V]; returns the number of produced tokens.
int sampled_accept(const float *lg, int V, const int32_t *draft, int nd, float temperature, StdRng &rng,
                   int32_t *out, int *accepted) {
  int acc = 0, prod = 0;
  for (int i = 0; i < nd; ++i) {
    const float *row = lg + (size_t)i * V;
    const int d = draft[i];
    const float pt = softmax_probabilities(row, V, temperature)[d];
    const float pd = 1.0f;  // point mass: one +inf among -inf
    const float ap = pd > 0.0f ? std::fmin(pt / pd, 1.0f) : (pt > 0.0f ? 1.0f : 0.0f);
    const float u = rng.gen_f32();
    if (u < ap) {
      out[prod++] = d;
      ++acc;
    } else {
      out[prod++] = sample_correction(row, V, d, temperature, rng);
      break;
    }
  }
  if (acc == nd) out[prod++] = sample_token(std::vector<float>(lg + (size_t)nd * V, lg + (size_t)(nd + 1) * V),
                                            temperature, rng);
  *accepted = acc;
  return prod;
}

// SpeculativeDecoder::step's phase 3 (speculative.rs:336-390): target rows
// [k + 1][V], the draft's logit rows [k][V] (as the draft produced them).
int spec_accept(const float *tl, const float *dl, int V, const int32_t *draft, int k, float temperature,
                StdRng &rng, int32_t *out, int *accepted) {
  int acc = 0, prod = 0;
  for (int i = 0; i < k; ++i) {
    const float *trow = tl + (size_t)i * V, *drow = dl + (size_t)i * V;
    const int d = draft[i];
    const float pt = softmax_probabilities(trow, V, temperature)[d];
    const float pd = softmax_probabilities(drow, V, temperature)[d];
    const float ap = pd > 0.0f ? std::fmin(pt / pd, 1.0f) : (pt > 0.0f ? 1.0f : 0.0f);
    const float u = rng.gen_f32();
    if (u < ap) {
      out[prod++] = d;
      ++acc;
    } else {
      // sample_correction with the draft's own distribution.
      const std::vector<float> tp = softmax_probabilities(trow, V, temperature);
      const std::vector<float> dp = softmax_probabilities(drow, V, temperature);
      double adj_sum = 0.0;
      std::vector<float> adj(V);
      for (int j = 0; j < V; ++j) {
        adj[j] = std::fmax(tp[j] - dp[j], 0.0f);
        adj_sum += (double)adj[j];
      }
      int tok = V - 1;
      if (!std::isfinite(adj_sum) || adj_sum <= 0.0) {
        tok = sample_token(std::vector<float>(trow, trow + V), temperature, rng);
      } else {
        const double uu = rng.gen_f64() * adj_sum;
        double cum = 0.0;
        for (int j = 0; j < V; ++j) {
          cum += (double)adj[j];
          if (cum >= uu) {
            tok = j;
            break;
          }
        }
      }
      out[prod++] = tok;
      break;
    }
  }
  if (acc == k) out[prod++] = sample_token(std::vector<float>(tl + (size_t)k * V, tl + (size_t)(k + 1) * V),
                                           temperature, rng);
  *accepted = acc;
  return prod;
}

int sampled_token(const float *lg, int V, float temperature, StdRng &rng) {
  return sample_token(std::vector<float>(lg, lg + V), temperature, rng);
}

}  // namespace ora

using namespace ora;

struct ora_rng {
  StdRng r;
};

extern "C" {

int ora_chacha_block(const uint32_t *key, uint64_t counter, uint64_t stream, int rounds, uint32_t *out) {
  ORA_TRY(chacha_block(key, counter, stream, rounds, out));
}

int ora_rng_create(uint64_t seed, int rounds, const uint32_t *key, ora_rng **out) {
  ORA_TRY({
    auto r = new ora_rng();
    if (key) {
      std::memcpy(r->r.key, key, 32);
      r->r.counter = 0;
      r->r.index = 64;
    } else {
      seed_from_u64(r->r, seed);
    }
    r->r.rounds = rounds;
    *out = r;
  });
}
void ora_rng_free(ora_rng *r) { delete r; }
uint32_t ora_rng_next_u32(ora_rng *r) { return r->r.next_u32(); }
uint64_t ora_rng_next_u64(ora_rng *r) { return r->r.next_u64(); }
float ora_rng_gen_f32(ora_rng *r) { return r->r.gen_f32(); }
double ora_rng_gen_f64(ora_rng *r) { return r->r.gen_f64(); }
float ora_standard_f32(uint32_t u) { return standard_f32(u); }
double ora_standard_f64(uint64_t u) { return standard_f64(u); }
void ora_rng_key(const ora_rng *r, uint32_t *key) { std::memcpy(key, r->r.key, 32); }

int ora_sample_token(const float *logits, int n, float temperature, ora_rng *r, int *token) {
  ORA_TRY(*token = sample_token(std::vector<float>(logits, logits + n), temperature, r->r));
}
int ora_sample_plain(const float *logits, int n, const int32_t *ctx, int len, float temperature, int64_t top_k,
                     float top_p, float penalty, ora_rng *r, int *token) {
  ORA_TRY(*token = sample_plain(logits, n, ctx, len, temperature, top_k, top_p, penalty, r->r));
}
int ora_softmax_probabilities(const float *logits, int n, float temperature, float *out) {
  ORA_TRY({
    const std::vector<float> p = softmax_probabilities(logits, n, temperature);
    std::memcpy(out, p.data(), sizeof(float) * n);
  });
}
int ora_sampled_accept(const float *lg, int V, const int32_t *draft, int nd, float temperature, ora_rng *r,
                       int32_t *out, int *produced, int *accepted) {
  ORA_TRY(*produced = sampled_accept(lg, V, draft, nd, temperature, r->r, out, accepted));
}
int ora_spec_accept(const float *tl, const float *dl, int V, const int32_t *draft, int k, float temperature,
                    ora_rng *r, int32_t *out, int *produced, int *accepted) {
  ORA_TRY(*produced = spec_accept(tl, dl, V, draft, k, temperature, r->r, out, accepted));
}

}  // extern "C"
