// Exact-sampling acceptance for prompt lookup (lookup.rs:359-403) and the
// sampled decode_one token (lookup.rs:428-455), on the device, drawing from
// the decoder's own rand 0.8 StdRng (ChaCha12, rand_chacha 0.3.1 over
// rand_core 0.6.4) so a step needs no host round trip and replays as part of
// the step graph.
//
// The reference's arithmetic is kept in its order: the softmax sums
// (f32, sequential over the vocabulary), the residual sum and its cumulative
// search (f64, sequential), the sample_token cumulative search (f32,
// sequential).  Those chains run in one wave (lane 0's order, values
// broadcast with readlane); everything order-free (scaling, maxima, the
// exponentials, the normalisation) runs on the whole block.  The draft rows'
// probabilities (softmax_probabilities: x / T, e / sum) are computed by
// k_sample_probs, one block per row, so their sum chains run in parallel;
// the bonus row uses sample_token's own variant (x * (1 / T), e * (1 / sum)).
//
// Generator: ChaCha block with 12 rounds, key from SeedableRng::seed_from_u64
// (set on the host), 64-bit block counter in words 12-13, stream 0; four
// blocks per refill; u32 draws in order; u64 = low word then high word,
// across a refill as BlockRng::next_u64 does; Standard f32 = (u32 >> 8) *
// 2^-24, f64 = (u64 >> 11) * 2^-53.
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>

#include "exact_math.h"
#include "kernels.h"

namespace rai {

namespace {

__device__ __forceinline__ uint32_t rotl32(uint32_t x, int r) { return (x << r) | (x >> (32 - r)); }

__device__ void chacha12(const uint32_t *key, uint64_t counter, uint32_t *out) {
  uint32_t in[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u};
  for (int i = 0; i < 8; ++i) in[4 + i] = key[i];
  in[12] = (uint32_t)counter;
  in[13] = (uint32_t)(counter >> 32);
  in[14] = 0u;
  in[15] = 0u;
  uint32_t s[16];
  for (int i = 0; i < 16; ++i) s[i] = in[i];
  auto qr = [&](int a, int b, int c, int d) {
    s[a] += s[b]; s[d] = rotl32(s[d] ^ s[a], 16);
    s[c] += s[d]; s[b] = rotl32(s[b] ^ s[c], 12);
    s[a] += s[b]; s[d] = rotl32(s[d] ^ s[a], 8);
    s[c] += s[d]; s[b] = rotl32(s[b] ^ s[c], 7);
  };
  for (int r = 0; r < 12; r += 2) {
    qr(0, 4, 8, 12);
    qr(1, 5, 9, 13);
    qr(2, 6, 10, 14);
    qr(3, 7, 11, 15);
    qr(0, 5, 10, 15);
    qr(1, 6, 11, 12);
    qr(2, 7, 8, 13);
    qr(3, 4, 9, 14);
  }
  for (int i = 0; i < 16; ++i) out[i] = s[i] + in[i];
}

// One thread drives the generator; the state lives in device memory.
struct Gen {
  RngState *st;
  __device__ void refill() {
    const uint64_t c = (uint64_t)st->counter_lo | ((uint64_t)st->counter_hi << 32);
    for (int b = 0; b < 4; ++b) chacha12(st->key, c + b, st->buf + 16 * b);
    const uint64_t n = c + 4;
    st->counter_lo = (uint32_t)n;
    st->counter_hi = (uint32_t)(n >> 32);
  }
  __device__ uint32_t next_u32() {
    if (st->index >= 64) {
      refill();
      st->index = 0;
    }
    return st->buf[st->index++];
  }
  __device__ uint64_t next_u64() {
    const int i = st->index;
    if (i < 63) {
      st->index = i + 2;
      return (uint64_t)st->buf[i] | ((uint64_t)st->buf[i + 1] << 32);
    }
    if (i >= 64) {
      refill();
      st->index = 2;
      return (uint64_t)st->buf[0] | ((uint64_t)st->buf[1] << 32);
    }
    const uint64_t lo = st->buf[63];
    refill();
    st->index = 1;
    return lo | ((uint64_t)st->buf[0] << 32);
  }
  __device__ float gen_f32() { return (float)(next_u32() >> 8) * (1.0f / 16777216.0f); }
  __device__ double gen_f64() { return (double)(next_u64() >> 11) * (1.0 / 9007199254740992.0); }
};

constexpr int kSampleThreads = 1024;
typedef float f4v __attribute__((ext_vector_type(4)));

// Sequential chains, block-wide calls.  The values pass through LDS in
// chunks of kStage; wave 0 walks a chunk with broadcast 16-byte reads (every
// lane computes the same chain, so the next reads issue while the adds
// wait on each other), which leaves one dependent add per element.
constexpr int kStage = 4096;

// f32 sum of p[0..n) from +0 in index order (every thread returns it).
// The values are >= +0, so padding with +0 changes nothing.
__device__ float seq_sum(const float *p, int n) {
  __shared__ __align__(16) float buf[kStage];
  __shared__ float res;
  float c = 0.0f;
  for (int c0 = 0; c0 < n; c0 += kStage) {
    const int cn = min(kStage, n - c0);
    __syncthreads();
    for (int i = threadIdx.x; i < kStage; i += blockDim.x) buf[i] = i < cn ? p[c0 + i] : 0.0f;
    __syncthreads();
    if (threadIdx.x < 64) {
      for (int i = 0; i < cn; i += 32) {
        f4v v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = *reinterpret_cast<const f4v *>(&buf[i + 4 * u]);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          c = c + v[u][0];
          c = c + v[u][1];
          c = c + v[u][2];
          c = c + v[u][3];
        }
      }
    }
  }
  if (threadIdx.x == 0) res = c;
  __syncthreads();
  return res;
}

// First i with r < p[0] + ... + p[i] (f32, index order); -1 if none.  Each
// 64-element block runs the chain alone; the values are >= +0, so the sums
// never decrease and a block holds the first hit only if its last sum is
// not <= r (a NaN sum also replays).  That block is replayed from its start
// with the running sums landing in lane k (off the chain), and one ballot
// finds the first hit.
__device__ int seq_search(const float *p, int n, float r) {
  __shared__ __align__(16) float buf[kStage];
  __shared__ int res;
  const int lane = threadIdx.x & 63;
  float c = 0.0f;
  int found = -1;
  for (int c0 = 0; c0 < n && found < 0; c0 += kStage) {
    const int cn = min(kStage, n - c0);
    __syncthreads();
    for (int i = threadIdx.x; i < kStage; i += blockDim.x) buf[i] = i < cn ? p[c0 + i] : 0.0f;
    __syncthreads();
    if (threadIdx.x < 64) {
      for (int i = 0; i < cn && found < 0; i += 64) {
        f4v v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = *reinterpret_cast<const f4v *>(&buf[i + 4 * u]);
        const float cstart = c;
#pragma unroll
        for (int u = 0; u < 16; ++u) {
#pragma unroll
          for (int w = 0; w < 4; ++w) c = c + v[u][w];
        }
        if (!(c <= r)) {
          float cc = cstart, pref = 0.0f;
#pragma unroll
          for (int u = 0; u < 16; ++u) {
#pragma unroll
            for (int w = 0; w < 4; ++w) {
              cc = cc + v[u][w];
              pref = lane == 4 * u + w ? cc : pref;
            }
          }
          const uint64_t hit = __ballot(r < pref && i + lane < cn);
          if (hit) found = c0 + i + __ffsll((unsigned long long)hit) - 1;
        }
      }
    }
    if (threadIdx.x == 0) res = found;
    __syncthreads();
    found = res;
  }
  return found;
}

// The residual max(0, p - q) of sample_correction as f64, q the draft's
// probabilities (pq) or the point mass on d.
__device__ __forceinline__ double residual(const float *pa, const float *pq, int d, int j) {
  const float q = pq ? pq[j] : (j == d ? 1.0f : 0.0f);
  return (double)fmaxf(pa[j] - q, 0.0f);
}

// f64 sum of the residuals over [0, n) from +0 in index order.
__device__ double seq_sum_resid(const float *pa, const float *pq, int d, int n) {
  __shared__ __align__(16) double buf[kStage];
  __shared__ double res;
  double c = 0.0;
  for (int c0 = 0; c0 < n; c0 += kStage) {
    const int cn = min(kStage, n - c0);
    __syncthreads();
    for (int i = threadIdx.x; i < kStage; i += blockDim.x) buf[i] = i < cn ? residual(pa, pq, d, c0 + i) : 0.0;
    __syncthreads();
    if (threadIdx.x < 64) {
      for (int i = 0; i < cn; i += 16) {
        double v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = buf[i + u];
#pragma unroll
        for (int u = 0; u < 16; ++u) c = c + v[u];
      }
    }
  }
  if (threadIdx.x == 0) res = c;
  __syncthreads();
  return res;
}

// First i with (residual[0] + ... + residual[i]) >= u (f64); n - 1 if none.
// As seq_search: the chain alone per 64-element block, the block whose last
// sum is not < u replayed for the first hit.
__device__ int seq_search_resid(const float *pa, const float *pq, int d, int n, double u) {
  __shared__ __align__(16) double buf[kStage];
  __shared__ int res;
  const int lane = threadIdx.x & 63;
  double c = 0.0;
  int found = -1;
  for (int c0 = 0; c0 < n && found < 0; c0 += kStage) {
    const int cn = min(kStage, n - c0);
    __syncthreads();
    for (int i = threadIdx.x; i < kStage; i += blockDim.x) buf[i] = i < cn ? residual(pa, pq, d, c0 + i) : 0.0;
    __syncthreads();
    if (threadIdx.x < 64) {
      for (int i = 0; i < cn && found < 0; i += 64) {
        const double cstart = c;
#pragma unroll
        for (int sb = 0; sb < 4; ++sb) {
          double v[16];
#pragma unroll
          for (int k = 0; k < 16; ++k) v[k] = buf[i + 16 * sb + k];
#pragma unroll
          for (int k = 0; k < 16; ++k) c = c + v[k];
        }
        if (!(c < u)) {
          double cc = cstart, pref = 0.0;
#pragma unroll
          for (int sb = 0; sb < 4; ++sb) {
            double v[16];
#pragma unroll
            for (int k = 0; k < 16; ++k) v[k] = buf[i + 16 * sb + k];
#pragma unroll
            for (int k = 0; k < 16; ++k) {
              cc = cc + v[k];
              pref = lane == 16 * sb + k ? cc : pref;
            }
          }
          const uint64_t hit = __ballot(pref >= u && i + lane < cn);
          if (hit) found = c0 + i + __ffsll((unsigned long long)hit) - 1;
        }
      }
    }
    if (threadIdx.x == 0) res = found;
    __syncthreads();
    found = res;
  }
  return found < 0 ? n - 1 : found;
}

// Block-wide reductions (every thread returns the result).
__device__ float block_max(float v, float *red) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); ++w) r = fmaxf(r, red[w]);
  return r;
}
__device__ int block_sum_i(int v, int *red) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  int r = 0;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) r += red[w];
  return r;
}

// Probabilities of one logit row into `out` (block-wide).  SAMPLE false:
// softmax_probabilities (speculative.rs:431-477): x / T, e / sum.  SAMPLE
// true: sample_token's softmax (sampler.rs:55-126, top_k = 0): NaN -> -inf,
// x * (1 / T), e * (1 / sum).  NaN scaled values are -inf in both.
template <bool SAMPLE>
__device__ void row_probs(const float *row, int V, float T, float *out, float *redf, int *redi) {
  const int tid = threadIdx.x, nt = blockDim.x;
  const float inv = 1.0f / T;
  int pinf = 0;
  float mx = -INFINITY;
  for (int i = tid; i < V; i += nt) {
    float x = row[i];
    if (SAMPLE) {
      if (isnan(x)) x = -INFINITY;
      x = x * inv;
    } else {
      x = x / T;
      if (isnan(x)) x = -INFINITY;
    }
    out[i] = x;
    pinf += x == INFINITY;
    mx = fmaxf(mx, x);
  }
  pinf = block_sum_i(pinf, redi);
  mx = block_max(mx, redf);
  if (pinf > 0) {
    const float p = 1.0f / (float)pinf;
    for (int i = tid; i < V; i += nt) out[i] = out[i] == INFINITY ? p : 0.0f;
    __syncthreads();
    return;
  }
  if (mx == -INFINITY) {
    for (int i = tid; i < V; i += nt) out[i] = 1.0f / (float)V;
    __syncthreads();
    return;
  }
  for (int i = tid; i < V; i += nt) out[i] = rai_exact::expf_glibc(out[i] - mx);
  __syncthreads();
  const float sum = seq_sum(out, V);
  if (!(isfinite(sum) && sum > 0.0f)) {
    for (int i = tid; i < V; i += nt) out[i] = 1.0f / (float)V;
  } else if (SAMPLE) {
    const float is = 1.0f / sum;
    for (int i = tid; i < V; i += nt) out[i] = out[i] * is;
  } else {
    for (int i = tid; i < V; i += nt) out[i] = out[i] / sum;
  }
  __syncthreads();
}

// argmax (sampler.rs:201-208): f32::total_cmp order, the last maximum wins
// (block-wide; every thread returns it).
__device__ int block_argmax(const float *p, int V) {
  __shared__ long long best[16];
  long long b = LLONG_MIN;
  for (int i = threadIdx.x; i < V; i += blockDim.x) {
    const int32_t bits = __float_as_int(p[i]);
    const int32_t key = bits ^ (int32_t)(((uint32_t)(bits >> 31)) >> 1);
    const long long k = ((long long)key << 32) | (uint32_t)i;
    b = k > b ? k : b;
  }
  for (int o = 32; o > 0; o >>= 1) {
    const long long x = __shfl_xor(b, o, 64);
    b = x > b ? x : b;
  }
  __syncthreads();
  if ((threadIdx.x & 63) == 0) best[threadIdx.x >> 6] = b;
  __syncthreads();
  long long r = best[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); ++w) r = best[w] > r ? best[w] : r;
  __syncthreads();
  return (int)(r & 0xFFFFFFFFll);
}

// sample_token's draw over the probabilities p (block-wide; thread 0 draws).
__device__ int draw_token(const float *p, int V, Gen &g, int *ires) {
  __shared__ float rr;
  if (threadIdx.x == 0) rr = g.gen_f32();
  __syncthreads();
  int tok = seq_search(p, V, rr);
  (void)ires;
  // Fallback: argmax of the probabilities.
  if (tok < 0) tok = block_argmax(p, V);
  return tok;
}

// Block per verify row: rows < nd get softmax_probabilities, row nd (the
// bonus row, or the decode_one row when nd = 0) sample_token's variant.
__global__ __launch_bounds__(kSampleThreads) void k_sample_probs(const float *__restrict__ logits, int V, int nd,
                                                                 float T, float *__restrict__ probs,
                                                                 const int *__restrict__ st) {
  __shared__ float redf[16];
  __shared__ int redi[16];
  if (st) {
    nd = st[3];
    T = __int_as_float(st[4]);
  }
  const int r = blockIdx.x;
  if (r > nd) return;
  if (r < nd)
    row_probs<false>(logits + (size_t)r * V, V, T, probs + (size_t)r * V, redf, redi);
  else
    row_probs<true>(logits + (size_t)r * V, V, T, probs + (size_t)r * V, redf, redi);
}

// lookup.rs:359-403 (and decode_one's sample when nd = 0).  Appends the
// produced tokens to ctx[len..] and writes res = {accepted, produced}.
// `scratch` holds V floats for the rare sample_token fallback of a
// correction.
// `pdraft` (may be null): the draft's own probabilities [nd][V]
// (SpeculativeDecoder, speculative.rs:336-370); null is prompt lookup's
// point mass on the drafted token.
__global__ __launch_bounds__(kSampleThreads) void k_sample_accept(
    const float *__restrict__ logits, const float *__restrict__ probs, const float *__restrict__ pdraft, int V,
    uint32_t *__restrict__ ctx, int len, int start, int nd, float T, RngState *rng, float *__restrict__ scratch,
    int *__restrict__ res, const int *__restrict__ st) {
  if (st) {
    len = st[1];
    start = st[2];
    nd = st[3];
    T = __int_as_float(st[4]);
  }
  Gen g{rng};
  __shared__ int sh_acc, sh_prod, sh_tok, sh_dec;
  __shared__ double sh_u;
  __shared__ float redf[16];
  __shared__ int redi[16];
  const int tid = threadIdx.x;
  if (tid == 0) {
    sh_acc = 0;
    sh_prod = 0;
  }
  __syncthreads();
  for (int i = 0; i < nd; ++i) {
    const float *pa = probs + (size_t)i * V;
    __syncthreads();  // every thread has read the previous decision
    if (tid == 0) {
      const int d = (int)ctx[start + i];
      const float pt = pa[d];
      const float pd = pdraft ? pdraft[(size_t)i * V + d] : 1.0f;  // point mass: 1
      const float ap = pd > 0.0f ? fminf(pt / pd, 1.0f) : (pt > 0.0f ? 1.0f : 0.0f);
      const float u = g.gen_f32();
      sh_dec = u < ap;
      if (sh_dec) {
        ctx[len + sh_prod] = (uint32_t)d;
        sh_prod = sh_prod + 1;
        sh_acc = sh_acc + 1;
      }
    }
    __syncthreads();
    if (sh_dec) continue;
    // sample_correction (speculative.rs:479-513): residual max(0, p - q)
    // with q the draft's distribution; sum and search in f64.
    const int d = (int)ctx[start + i];
    const float *pq = pdraft ? pdraft + (size_t)i * V : nullptr;
    const double as = seq_sum_resid(pa, pq, d, V);
    if (!(isfinite(as) && as > 0.0)) {
      // sample_token over the target row (unreachable when the draft's
      // probability is below 1; kept for the reference's semantics).
      row_probs<true>(logits + (size_t)i * V, V, T, scratch, redf, redi);
      const int tok = draw_token(scratch, V, g, &sh_tok);
      if (tid == 0) sh_tok = tok;
    } else {
      if (tid == 0) sh_u = g.gen_f64() * as;
      __syncthreads();
      const int tok = seq_search_resid(pa, pq, d, V, sh_u);
      if (tid == 0) sh_tok = tok;
    }
    __syncthreads();
    if (tid == 0) {
      ctx[len + sh_prod] = (uint32_t)sh_tok;
      sh_prod = sh_prod + 1;
    }
    __syncthreads();
    break;
  }
  __syncthreads();
  if (sh_acc == nd) {
    const int tok = draw_token(probs + (size_t)nd * V, V, g, &sh_tok);
    if (tid == 0) {
      ctx[len + sh_prod] = (uint32_t)tok;
      sh_prod = sh_prod + 1;
    }
  }
  __syncthreads();
  if (tid == 0) {
    res[0] = sh_acc;
    res[1] = sh_prod;
  }
}

// One draft token of SpeculativeDecoder::step (speculative.rs:246-271):
// the row is kept in `keep` (for p_draft), then sample_token draws *out.
__global__ __launch_bounds__(kSampleThreads) void k_draw(const float *__restrict__ row, int V, float T,
                                                         RngState *rng, float *__restrict__ keep,
                                                         float *__restrict__ scratch, uint32_t *out) {
  __shared__ float redf[16];
  __shared__ int redi[16];
  __shared__ int tok;
  for (int i = threadIdx.x; i < V; i += blockDim.x) keep[i] = row[i];
  Gen g{rng};
  row_probs<true>(row, V, T, scratch, redf, redi);
  const int t = draw_token(scratch, V, g, &tok);
  if (threadIdx.x == 0) *out = (uint32_t)t;
}

// Device draws for a check against the CPU restatement: kinds[i] 0 = u32,
// 1 = u64, 2 = f32, 3 = f64; out[i] holds the raw bits (64-bit).
__global__ void k_rng_draws(RngState *rng, const int *kinds, int n, uint64_t *out) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  Gen g{rng};
  for (int i = 0; i < n; ++i) {
    switch (kinds[i]) {
      case 0: out[i] = g.next_u32(); break;
      case 1: out[i] = g.next_u64(); break;
      case 2: out[i] = (uint64_t)__float_as_uint(g.gen_f32()); break;
      default: out[i] = __builtin_bit_cast(uint64_t, g.gen_f64()); break;
    }
  }
}

// ------------------------------------------------------------ plain sampler --
//
// apply_repetition_penalty (sampler.rs:185-199) over ctx[0..len), then
// sample_token (sampler.rs:47-182) with the whole SamplerConfig: the token
// of the `rai run` loop without speculation (run.rs:720-721).  One block of
// kSampleThreads; x [V] is the working row, flags [V] are zero on entry and
// on exit (they mark the penalised tokens, then the top-p nucleus).

// f32::total_cmp order as an unsigned key, and back.
__device__ __forceinline__ uint32_t total_key(float v) {
  const uint32_t b = __float_as_uint(v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float total_val(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// Block-wide exclusive prefix sum of one count per thread; *total gets the
// block's sum.
__device__ int block_excl_scan(int v, int *total) {
  __shared__ int wsum[16];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int inc = v;
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(inc, o, 64);
    if (lane >= o) inc += y;
  }
  __syncthreads();
  if (lane == 63) wsum[w] = inc;
  __syncthreads();
  int base = 0, tot = 0;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) {
    if (i < w) base += wsum[i];
    tot += wsum[i];
  }
  *total = tot;
  return base + inc - v;
}

// Stage chunk [c0, c0 + cn) of x compactly in index order: its non-zero
// values to vbuf (and their indices to ibuf), padded with +0 to a multiple
// of 64; returns the count.  (kStage = 4 x kSampleThreads.)
__device__ int stage_nonzero(const float *x, int c0, int cn, float *vbuf, int *ibuf) {
  float v[4];
  int k = 0;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int i = 4 * threadIdx.x + u;
    v[u] = i < cn ? x[c0 + i] : 0.0f;
    k += v[u] != 0.0f;
  }
  int tot;
  int o = block_excl_scan(k, &tot);
#pragma unroll
  for (int u = 0; u < 4; ++u)
    if (v[u] != 0.0f) {
      vbuf[o] = v[u];
      if (ibuf) ibuf[o] = c0 + 4 * threadIdx.x + u;
      ++o;
    }
  const int padded = (tot + 63) & ~63;
  for (int i = tot + threadIdx.x; i < padded; i += blockDim.x) vbuf[i] = 0.0f;
  __syncthreads();
  return tot;
}

// seq_sum over the non-zero entries only: the values are >= +0, so adding
// a zero leaves every partial sum unchanged.
__device__ float seq_sum_nz(const float *x, int n) {
  __shared__ __align__(16) float buf[kStage];
  __shared__ float res;
  float c = 0.0f;
  for (int c0 = 0; c0 < n; c0 += kStage) {
    const int tot = stage_nonzero(x, c0, min(kStage, n - c0), buf, nullptr);
    if (threadIdx.x < 64) {
      for (int i = 0; i < tot; i += 32) {
        f4v v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = *reinterpret_cast<const f4v *>(&buf[i + 4 * u]);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          c = c + v[u][0];
          c = c + v[u][1];
          c = c + v[u][2];
          c = c + v[u][3];
        }
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) res = c;
  __syncthreads();
  return res;
}

// seq_search over the non-zero entries only: the running sum does not move
// at a zero entry, so the first index where r < sum is a non-zero one.
__device__ int seq_search_nz(const float *x, int n, float r) {
  __shared__ __align__(16) float buf[kStage];
  __shared__ int bidx[kStage];
  __shared__ int res;
  const int lane = threadIdx.x & 63;
  float c = 0.0f;
  int found = -1;
  for (int c0 = 0; c0 < n && found < 0; c0 += kStage) {
    const int tot = stage_nonzero(x, c0, min(kStage, n - c0), buf, bidx);
    if (threadIdx.x < 64) {
      for (int i = 0; i < tot && found < 0; i += 64) {
        f4v v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = *reinterpret_cast<const f4v *>(&buf[i + 4 * u]);
        const float cstart = c;
#pragma unroll
        for (int u = 0; u < 16; ++u) {
#pragma unroll
          for (int w = 0; w < 4; ++w) c = c + v[u][w];
        }
        if (!(c <= r)) {
          float cc = cstart, pref = 0.0f;
#pragma unroll
          for (int u = 0; u < 16; ++u) {
#pragma unroll
            for (int w = 0; w < 4; ++w) {
              cc = cc + v[u][w];
              pref = lane == 4 * u + w ? cc : pref;
            }
          }
          const uint64_t hit = __ballot(r < pref && i + lane < tot);
          if (hit) found = bidx[i + __ffsll((unsigned long long)hit) - 1];
        }
      }
    }
    if (threadIdx.x == 0) res = found;
    __syncthreads();
    found = res;
  }
  return found;
}

// The key of descending rank `rank` (0-based) under total_cmp among the
// entries i of x with elig(i) (rank < their count): a four-pass radix
// selection over the key bytes.  *eq_before: how many entries with that key
// rank before it (so rank - *eq_before entries have larger keys).
template <class E>
__device__ uint32_t select_desc(const float *x, int V, int rank, E elig, int *eq_before) {
  __shared__ unsigned hist[256];
  __shared__ uint32_t sh_prefix;
  __shared__ int sh_rank;
  uint32_t prefix = 0, hmask = 0;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = threadIdx.x; i < 256; i += blockDim.x) hist[i] = 0u;
    __syncthreads();
    for (int i = threadIdx.x; i < V; i += blockDim.x)
      if (elig(i)) {
        const uint32_t k = total_key(x[i]);
        if ((k & hmask) == prefix) atomicAdd(&hist[(k >> shift) & 255u], 1u);
      }
    __syncthreads();
    if (threadIdx.x == 0) {
      int r = rank, d = 255;
      for (; d > 0; --d) {
        if (r < (int)hist[d]) break;
        r -= (int)hist[d];
      }
      sh_prefix = prefix | ((uint32_t)d << shift);
      sh_rank = r;
    }
    __syncthreads();
    prefix = sh_prefix;
    rank = sh_rank;
    hmask |= 255u << shift;
  }
  *eq_before = rank;
  return prefix;
}

// Top-p (sampler.rs:129-167) over the probabilities x: the candidates
// p > 1e-10 in descending p (ties lowest index first), the shortest prefix
// whose f32 running sum from +0 reaches tp, everything else zeroed, then the
// division by the f32 sum in index order.  The candidates are taken 1024 at
// a time: the 1024 largest not taken yet (a radix selection, equal keys by
// index), sorted in LDS (bitonic), and thread 0 continues the running sum
// over them in order; the taken ones are marked 2 in flags.
__device__ void top_p_nucleus(float *x, int V, float tp, uint32_t *flags, int *redi) {
  constexpr int B = kSampleThreads;
  __shared__ uint32_t skey[B];
  __shared__ int sidx[B];
  __shared__ int sh_cnt, sh_cut, sh_done;
  __shared__ float sh_cum;
  const int tid = threadIdx.x, nt = blockDim.x;
  auto cand = [&](int i) { return x[i] > 1e-10f && flags[i] != 2u; };
  int remaining = 0;
  for (int i = tid; i < V; i += nt) remaining += cand(i);
  remaining = block_sum_i(remaining, redi);
  if (tid == 0) sh_cum = 0.0f;
  bool done = false;
  while (!done && remaining > 0) {
    const int take = min(B, remaining);
    const bool all = take == remaining;
    uint32_t kth = 0;
    int need_eq = 0;
    if (!all) {
      int before;
      kth = select_desc(x, V, take - 1, cand, &before);
      need_eq = before + 1;
    }
    if (tid == 0) sh_cnt = 0;
    for (int i = tid; i < B; i += nt) {
      skey[i] = 0u;
      sidx[i] = INT_MAX;
    }
    __syncthreads();
    for (int i = tid; i < V; i += nt)
      if (cand(i)) {
        const uint32_t k = total_key(x[i]);
        if (all || k > kth) {
          const int slot = atomicAdd(&sh_cnt, 1);
          skey[slot] = k;
          sidx[slot] = i;
        }
      }
    __syncthreads();
    if (!all) {
      // The entries equal to the k-th key, lowest index first.
      int got = 0;
      for (int c0 = 0; c0 < V && got < need_eq; c0 += nt) {
        const int i = c0 + tid;
        const int eq = i < V && cand(i) && total_key(x[i]) == kth;
        int tot;
        const int off = block_excl_scan(eq, &tot);
        if (eq && got + off < need_eq) {
          skey[take - need_eq + got + off] = kth;
          sidx[take - need_eq + got + off] = i;
        }
        got += tot;
      }
      __syncthreads();
    }
    // Bitonic sort: descending key, then ascending index.
    for (int k = 2; k <= B; k <<= 1)
      for (int j = k >> 1; j > 0; j >>= 1) {
        const int i = tid, ixj = i ^ j;
        if (ixj > i) {
          const uint32_t ka = skey[i], kb = skey[ixj];
          const int ia = sidx[i], ib = sidx[ixj];
          const bool a_first = ka > kb || (ka == kb && ia < ib);
          const bool up = (i & k) == 0;
          if (up ? !a_first : a_first) {
            skey[i] = kb;
            skey[ixj] = ka;
            sidx[i] = ib;
            sidx[ixj] = ia;
          }
        }
        __syncthreads();
      }
    if (tid == 0) {
      float c = sh_cum;
      int cut = take, fin = 0;
      for (int j = 0; j < take; ++j) {
        c = c + total_val(skey[j]);
        if (c >= tp) {
          cut = j + 1;
          fin = 1;
          break;
        }
      }
      sh_cum = c;
      sh_cut = cut;
      sh_done = fin;
    }
    __syncthreads();
    for (int j = tid; j < sh_cut; j += nt) flags[sidx[j]] = 2u;
    __syncthreads();
    done = sh_done != 0;
    remaining -= take;
  }
  for (int i = tid; i < V; i += nt) {
    const bool keep = flags[i] == 2u;
    x[i] = keep ? x[i] : 0.0f;
    flags[i] = 0u;
  }
  __syncthreads();
  const float sum = seq_sum_nz(x, V);
  if (sum > 0.0f) {
    const float is = 1.0f / sum;
    for (int i = tid; i < V; i += nt) x[i] = x[i] * is;
  }
  __syncthreads();
}

// The plain token: writes it to tok_out (ctx + len when null) and, when res
// is given, res = {0 accepted, 1 produced}.  With a step record, len, T and
// the sampler options come from st[1], st[4], st[8..10].
__global__ __launch_bounds__(kSampleThreads) void k_sample_plain(
    const float *__restrict__ logits, int V, uint32_t *__restrict__ ctx, int len, float T, int top_k, float top_p,
    float pen, RngState *rng, float *__restrict__ x, uint32_t *__restrict__ flags, uint32_t *tok_out, int *res,
    const int *__restrict__ st) {
  if (st) {
    len = st[1];
    T = __int_as_float(st[4]);
    top_k = st[8];
    top_p = __int_as_float(st[9]);
    pen = __int_as_float(st[10]);
  }
  __shared__ float redf[16];
  __shared__ int redi[16];
  __shared__ float rr;
  const int tid = threadIdx.x, nt = blockDim.x;
  // apply_repetition_penalty: each distinct token once.
  const bool penal = isfinite(pen) && pen > 0.0f && fabsf(pen - 1.0f) >= 1e-6f;
  if (penal)
    for (int i = tid; i < len; i += nt) {
      const uint32_t t = ctx[i];
      if (t < (uint32_t)V) flags[t] = 1u;
    }
  __syncthreads();
  for (int i = tid; i < V; i += nt) {
    float v = logits[i];
    if (penal && flags[i]) {
      v = v > 0.0f ? v / pen : v * pen;
      flags[i] = 0u;
    }
    x[i] = isnan(v) ? -INFINITY : v;
  }
  __syncthreads();
  int tok;
  if (!isfinite(T) || T <= 1e-6f) {
    tok = block_argmax(x, V);
  } else {
    const float inv_t = 1.0f / T;
    for (int i = tid; i < V; i += nt) x[i] = x[i] * inv_t;
    __syncthreads();
    if (top_k > 0 && top_k < V) {
      int before;
      const float thr = total_val(select_desc(x, V, top_k - 1, [](int) { return true; }, &before));
      for (int i = tid; i < V; i += nt)
        if (x[i] < thr) x[i] = -INFINITY;
      __syncthreads();
    }
    int pinf = 0;
    float mx = -INFINITY;
    for (int i = tid; i < V; i += nt) {
      pinf += x[i] == INFINITY;
      mx = fmaxf(mx, x[i]);
    }
    pinf = block_sum_i(pinf, redi);
    mx = block_max(mx, redf);
    if (pinf > 0) {
      const float p = 1.0f / (float)pinf;
      for (int i = tid; i < V; i += nt) x[i] = x[i] == INFINITY ? p : 0.0f;
    } else if (mx == -INFINITY) {
      for (int i = tid; i < V; i += nt) x[i] = 1.0f / (float)V;
    } else {
      for (int i = tid; i < V; i += nt) x[i] = rai_exact::expf_glibc(x[i] - mx);
      __syncthreads();
      const float sum = seq_sum_nz(x, V);
      if (isfinite(sum) && sum > 0.0f) {
        const float is = 1.0f / sum;
        for (int i = tid; i < V; i += nt) x[i] = x[i] * is;
      } else {
        for (int i = tid; i < V; i += nt) x[i] = 1.0f / (float)V;
      }
    }
    __syncthreads();
    const float tp = isfinite(top_p) ? fminf(fmaxf(top_p, 0.0f), 1.0f) : 1.0f;
    if (tp < 1.0f) top_p_nucleus(x, V, tp, flags, redi);
    if (tid == 0) {
      Gen g{rng};
      rr = g.gen_f32();
    }
    __syncthreads();
    tok = seq_search_nz(x, V, rr);
    if (tok < 0) tok = block_argmax(x, V);
  }
  if (tid == 0) {
    uint32_t *o = tok_out ? tok_out : ctx + len;
    *o = (uint32_t)tok;
    if (res) {
      res[0] = 0;
      res[1] = 1;
    }
  }
}

}  // namespace

void rng_seed_from_u64(RngState &r, uint64_t state) {
  // SeedableRng::seed_from_u64 (rand_core 0.6.4): PCG32 steps fill the key.
  const uint64_t mul = 6364136223846793005ull, inc = 11634580027462260723ull;
  for (int i = 0; i < 8; ++i) {
    state = state * mul + inc;
    const uint32_t xs = (uint32_t)(((state >> 18) ^ state) >> 27);
    const uint32_t rot = (uint32_t)(state >> 59);
    r.key[i] = (xs >> rot) | (xs << ((32 - rot) & 31));
  }
  r.counter_lo = r.counter_hi = 0;
  r.index = 64;
  for (uint32_t &w : r.buf) w = 0;
}

void launch_sample(const float *logits, float *probs, int V, uint32_t *ctx, int len, int start, int nd, float T,
                   RngState *rng, float *scratch, int *res, hipStream_t s, const int *st, int rows) {
  hipLaunchKernelGGL(k_sample_probs, dim3(rows), dim3(kSampleThreads), 0, s, logits, V, nd, T, probs, st);
  hipLaunchKernelGGL(k_sample_accept, dim3(1), dim3(kSampleThreads), 0, s, logits, probs, (const float *)nullptr,
                     V, ctx, len, start, nd, T, rng, scratch, res, st);
}

void launch_spec_sample(const float *tlogits, float *tprobs, const float *dlogits, float *dprobs, int V,
                        uint32_t *toks, int k, float T, RngState *rng, float *scratch, int *res, hipStream_t s) {
  hipLaunchKernelGGL(k_sample_probs, dim3(k + 1), dim3(kSampleThreads), 0, s, tlogits, V, k, T, tprobs,
                     (const int *)nullptr);
  if (k > 0)
    hipLaunchKernelGGL(k_sample_probs, dim3(k), dim3(kSampleThreads), 0, s, dlogits, V, k, T, dprobs,
                       (const int *)nullptr);
  hipLaunchKernelGGL(k_sample_accept, dim3(1), dim3(kSampleThreads), 0, s, tlogits, tprobs,
                     (const float *)dprobs, V, toks, k + 1, 1, k, T, rng, scratch, res, (const int *)nullptr);
}

void launch_draw(const float *row, int V, float T, RngState *rng, float *keep, float *scratch, uint32_t *out,
                 hipStream_t s) {
  hipLaunchKernelGGL(k_draw, dim3(1), dim3(kSampleThreads), 0, s, row, V, T, rng, keep, scratch, out);
}

void launch_sample_plain(const float *logits, int V, uint32_t *ctx, int len, float T, int top_k, float top_p,
                         float penalty, RngState *rng, float *work, uint32_t *flags, uint32_t *tok_out, int *res,
                         hipStream_t s, const int *st) {
  hipLaunchKernelGGL(k_sample_plain, dim3(1), dim3(kSampleThreads), 0, s, logits, V, ctx, len, T, top_k, top_p,
                     penalty, rng, work, flags, tok_out, res, st);
}

void launch_rng_draws(RngState *rng, const int *kinds, int n, uint64_t *out, hipStream_t s) {
  hipLaunchKernelGGL(k_rng_draws, dim3(1), dim3(64), 0, s, rng, kinds, n, out);
}

}  // namespace rai
