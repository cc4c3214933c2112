// Synthetic .raimodel writer: random-init models in the reference's byte
// layout (rai-infer/scripts/raimodel.py:485-615 packing, format.rs layout).
//
// Weight sources:
//   mode 0 / 1: N(0, weight_std) from a counter-based generator (splitmix64
//               + Box-Muller in double), so any tensor slice can be produced
//               in parallel and reproduced exactly;
//   mode 2:     the 64-bit LCG of gen_convert_fixture.py:53-71, walked in the
//               fixture's tensor order (reproduces tiny-convert.raimodel).
// Quantizers:
//   mode 0:     symmetric int4 RTN, scale = f16(absmax/7), q = clamp(rne(w/s),
//               -8, 7), stored code = q + 8, zero = -8*scale (exact in f16);
//   mode 1, 2:  the exporter's asymmetric min/max RTN (raimodel.py:257-303).
// The embedding is always 8-bit min/max RTN (quantize_embedding_8bit).
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

#include "common.h"
#include "format.h"

namespace rai {

// A synthetic image in malloc'd memory (freed with std::free).
struct SynthImage {
  uint8_t *data = nullptr;
  size_t size = 0;
};

namespace {

constexpr double kMinF16Scale = 5.9604644775390625e-08;  // 2^-24 (raimodel.py:65)

// IEEE binary16 from double, round to nearest even (numpy's astype(float16)).
uint16_t f64_to_f16(double v) {
  uint64_t b;
  std::memcpy(&b, &v, 8);
  const uint16_t sign = (uint16_t)((b >> 48) & 0x8000u);
  const double a = std::fabs(v);
  if (std::isnan(v)) return (uint16_t)(sign | 0x7E00u);
  if (a >= 65520.0) return (uint16_t)(sign | 0x7C00u);  // rounds to inf
  if (a < 5.9604644775390625e-08 / 2) {                  // below half the smallest subnormal
    if (a == 5.9604644775390625e-08 / 2) return sign;    // tie rounds to even (0)
    return sign;
  }
  int e;
  std::frexp(a, &e);  // a = f * 2^e, f in [0.5, 1)
  int exp16 = e - 1 + 15;
  double quantum;
  if (exp16 <= 0) {
    quantum = std::ldexp(1.0, -24);  // subnormal spacing
    exp16 = 0;
  } else {
    quantum = std::ldexp(1.0, e - 1 - 10);
  }
  double q = std::nearbyint(a / quantum);  // exact division by a power of two; RNE
  uint32_t mant = (uint32_t)q;
  if (exp16 == 0) {
    if (mant >= 1024) return (uint16_t)(sign | 0x0400u | (mant - 1024));  // rounded up to normal
    return (uint16_t)(sign | mant);
  }
  if (mant >= 2048) {  // rounding carried into the next binade
    mant >>= 1;
    ++exp16;
  }
  if (exp16 >= 31) return (uint16_t)(sign | 0x7C00u);
  return (uint16_t)(sign | (exp16 << 10) | (mant - 1024));
}

uint64_t splitmix(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

// Element i of tensor `tid`: N(0, std) via Box-Muller on a counter hash.
float gauss(uint64_t seed, uint64_t tid, uint64_t i, float stdv) {
  const uint64_t h = splitmix(seed ^ splitmix(tid * 0x100000001B3ull + (i >> 1)));
  const uint64_t h2 = splitmix(h);
  const double u1 = ((h >> 11) + 1.0) * (1.0 / 9007199254740993.0);  // (0, 1]
  const double u2 = (h2 >> 11) * (1.0 / 9007199254740992.0);         // [0, 1)
  const double r = std::sqrt(-2.0 * std::log(u1));
  const double z = (i & 1) ? r * std::sin(6.283185307179586 * u2) : r * std::cos(6.283185307179586 * u2);
  return (float)(stdv * z);
}

struct Lcg {  // gen_convert_fixture.py:53-71
  uint64_t state;
  uint32_t next() {
    state = state * 6364136223846793005ull + 1442695040888963407ull;
    return (uint32_t)(state >> 33);
  }
  float weight() { return (float)(((double)(next() % 4001) - 2000.0) / 4096.0); }
  float norm() { return (float)(1.0 + ((double)(next() % 201) - 100.0) / 1024.0); }
};

// Asymmetric min/max params for one row group (compute_group_params).
void minmax_params(const float *w, int n, int levels, uint16_t &s16, uint16_t &z16, double &s64,
                   double &z64) {
  double mn = w[0], mx = w[0];
  for (int i = 1; i < n; ++i) {
    mn = std::min(mn, (double)w[i]);
    mx = std::max(mx, (double)w[i]);
  }
  const double scale = std::max((mx - mn) / (levels - 1), kMinF16Scale);
  s16 = f64_to_f16(scale);
  z16 = f64_to_f16(mn);
  s64 = f16_bits_to_f32(s16);
  z64 = f16_bits_to_f32(z16);
}

int synth_threads() { return std::max(1, std::min<int>((int)std::thread::hardware_concurrency(), 16)); }

// fn(r0, r1) over [0, rows) split across the worker threads.
template <class F>
void parallel_rows(size_t rows, F fn) {
  const int nt = (int)std::min<size_t>(synth_threads(), std::max<size_t>(rows, 1));
  std::vector<std::thread> th;
  for (int i = 0; i < nt; ++i) th.emplace_back(fn, rows * i / nt, rows * (i + 1) / nt);
  for (auto &t : th) t.join();
}

// The weights of one tensor, row by row: N(0, std) from the counter hash
// (element j = r * cols + c of tensor `tid`; pairs of elements share one
// Box-Muller draw, so both come from one log / sqrt / sincos), or rows of a
// tensor generated up front (the fixture LCG).
struct Source {
  uint64_t seed = 0, tid = 0;
  float stdv = 0.0f;
  const float *pre = nullptr;  // pre-generated [rows][cols], or null
  void row(size_t r, size_t cols, float *out) const {
    if (pre) {
      std::memcpy(out, pre + r * cols, cols * sizeof(float));
      return;
    }
    size_t j = r * cols, c = 0;
    if (j & 1) out[c++] = gauss(seed, tid, j++, stdv);
    for (; c + 1 < cols; c += 2, j += 2) {
      const uint64_t h = splitmix(seed ^ splitmix(tid * 0x100000001B3ull + (j >> 1)));
      const uint64_t h2 = splitmix(h);
      const double u1 = ((h >> 11) + 1.0) * (1.0 / 9007199254740993.0);
      const double u2 = (h2 >> 11) * (1.0 / 9007199254740992.0);
      const double rr = std::sqrt(-2.0 * std::log(u1));
      out[c] = (float)(stdv * (rr * std::cos(6.283185307179586 * u2)));
      out[c + 1] = (float)(stdv * (rr * std::sin(6.283185307179586 * u2)));
    }
    if (c < cols) out[c] = gauss(seed, tid, j, stdv);
  }
};

// Bytes of one linear record ([u32 rows][u32 cols][params][nibbles],
// raimodel.py:518-526).
size_t linear_bytes(size_t rows, size_t cols, int gs) {
  return 8 + rows * ((cols + gs - 1) / gs) * 4 + rows * cols / 2;
}

// Quantize a [rows][cols] weight matrix row by row into its linear record at
// dst (int4 codes, symmetric or min/max RTN per group).
void put_linear(uint8_t *dst, const Source &src, int rows, int cols, int gs, bool sym) {
  if (cols % 2) fail(RAI_E_ARG, "synthetic linear needs an even column count");
  const int groups = (cols + gs - 1) / gs;
  const uint32_t hdr[2] = {(uint32_t)rows, (uint32_t)cols};
  std::memcpy(dst, hdr, 8);
  uint8_t *params = dst + 8;
  uint8_t *nib = params + (size_t)rows * groups * 4;
  parallel_rows(rows, [&](size_t r0, size_t r1) {
    std::vector<float> row(cols);
    std::vector<uint8_t> codes(cols);
    for (size_t r = r0; r < r1; ++r) {
      src.row(r, cols, row.data());
      for (int g = 0; g < groups; ++g) {
        const int c0 = g * gs, c1 = std::min(cols, c0 + gs);
        uint16_t s16, z16;
        double s64, z64;
        if (sym) {
          double am = 0.0;
          for (int c = c0; c < c1; ++c) am = std::max(am, std::fabs((double)row[c]));
          s16 = f64_to_f16(std::max(am / 7.0, kMinF16Scale));
          s64 = f16_bits_to_f32(s16);
          z16 = f64_to_f16(-8.0 * s64);
          for (int c = c0; c < c1; ++c) {
            const double q = std::min(7.0, std::max(-8.0, std::nearbyint((double)row[c] / s64)));
            codes[c] = (uint8_t)((int)q + 8);
          }
        } else {
          minmax_params(row.data() + c0, c1 - c0, 16, s16, z16, s64, z64);
          for (int c = c0; c < c1; ++c) {
            const double q = std::min(15.0, std::max(0.0, std::nearbyint(((double)row[c] - z64) / s64)));
            codes[c] = (uint8_t)q;
          }
        }
        const uint16_t p2[2] = {s16, z16};
        std::memcpy(params + (r * groups + g) * 4, p2, 4);
      }
      uint8_t *nr = nib + r * (size_t)cols / 2;
      for (int i = 0; i < cols / 2; ++i) nr[i] = (uint8_t)((codes[2 * i] & 0x0F) | ((codes[2 * i + 1] & 0x0F) << 4));
    }
  });
}

// The 8-bit min/max embedding (quantize_embedding_8bit): params
// [vocab][groups] x (scale, zero) f16, then codes [vocab][hidden].
size_t embedding_bytes(size_t vocab, size_t hidden, int egs) {
  return vocab * ((hidden + egs - 1) / egs) * 4 + vocab * hidden;
}

void put_embedding(uint8_t *dst, const Source &src, int vocab, int hidden, int egs) {
  const int groups = (hidden + egs - 1) / egs;
  uint8_t *params = dst;
  uint8_t *codes = dst + (size_t)vocab * groups * 4;
  parallel_rows(vocab, [&](size_t v0, size_t v1) {
    std::vector<float> row(hidden);
    for (size_t v = v0; v < v1; ++v) {
      src.row(v, hidden, row.data());
      for (int g = 0; g < groups; ++g) {
        const int c0 = g * egs, c1 = std::min(hidden, c0 + egs);
        uint16_t s16, z16;
        double s64, z64;
        minmax_params(row.data() + c0, c1 - c0, 256, s16, z16, s64, z64);
        const uint16_t p2[2] = {s16, z16};
        std::memcpy(params + (v * groups + g) * 4, p2, 4);
        for (int c = c0; c < c1; ++c) {
          const double q = std::min(255.0, std::max(0.0, std::nearbyint(((double)row[c] - z64) / s64)));
          codes[v * hidden + c] = (uint8_t)q;
        }
      }
    }
  });
}

// A raw f32 tensor (router) or a norm vector of ones.
void put_f32(uint8_t *dst, const Source &src, int rows, int cols) {
  parallel_rows(rows, [&](size_t r0, size_t r1) {
    for (size_t r = r0; r < r1; ++r) src.row(r, cols, reinterpret_cast<float *>(dst) + r * cols);
  });
}

}  // namespace

// The image is assembled in place: the section sizes follow from the shape,
// so one buffer is allocated and every tensor is quantized straight into its
// slot, row by row on the worker threads.  Tensor ids (the generator's
// streams) are taken in file order, as the reference exporter writes them.
SynthImage synth_model(const rai_synth_config &c, uint64_t seed) {
  if (c.mode > 2) fail(RAI_E_ARG, "unknown synth mode");
  if (c.num_experts != 0 && c.mode == 2) fail(RAI_E_ARG, "the LCG fixture mode is dense only");
  const int H = c.hidden_size, F = c.intermediate_size, V = c.vocab_size, L = c.num_layers;
  const int qd = c.num_heads * c.head_dim, kvd = c.num_kv_heads * c.head_dim;
  const int gs = c.group_size, egs = c.embed_group_size;
  if (H <= 0 || F <= 0 || V <= 0 || L <= 0 || gs <= 0 || egs <= 0 || c.num_kv_heads == 0)
    fail(RAI_E_ARG, "invalid synthetic model shape");
  const bool sym = c.mode == 0;
  const bool v2 = c.num_experts > 0;
  const int dims[7][2] = {{qd, H}, {kvd, H}, {kvd, H}, {H, qd}, {F, H}, {F, H}, {H, F}};
  // Section sizes.
  std::vector<size_t> sec;
  sec.push_back(embedding_bytes(V, H, egs));
  size_t layer = 0;
  for (int p = 0; p < 7; ++p) layer += linear_bytes(dims[p][0], dims[p][1], gs);
  if (v2) {
    layer += (size_t)c.num_experts * H * 4;
    for (uint32_t e = 1; e < c.num_experts; ++e)
      for (int p = 4; p < 7; ++p) layer += linear_bytes(dims[p][0], dims[p][1], gs);
  }
  layer += 2 * (size_t)H * 4;
  for (int l = 0; l < L; ++l) sec.push_back(layer);
  sec.push_back((size_t)H * 4);
  if (!c.tied) sec.push_back(linear_bytes(V, H, gs));
  const size_t hsz = v2 ? 128 : 64;
  size_t total = hsz + sec.size() * 16;
  for (size_t b : sec) total += b;
  SynthImage img;
  img.data = static_cast<uint8_t *>(std::malloc(total));
  if (!img.data) fail(RAI_E_OOM, "image allocation failed");
  img.size = total;
  uint8_t *const out = img.data;
  try {
    // Header (raimodel.py:558-579; v2 capability block per format.rs:21-40).
    std::memset(out, 0, hsz);
    std::memcpy(out, "RAIM", 4);
    auto put32 = [&](size_t off, uint32_t v) { std::memcpy(out + off, &v, 4); };
    auto putf = [&](size_t off, float v) { std::memcpy(out + off, &v, 4); };
    put32(4, v2 ? 2 : 1);
    put32(8, H);
    put32(12, L);
    put32(16, c.num_heads);
    put32(20, c.num_kv_heads);
    put32(24, c.head_dim);
    put32(28, F);
    put32(32, V);
    put32(36, c.max_context);
    putf(40, c.rope_theta);
    putf(44, c.norm_eps);
    out[48] = 4;
    out[49] = (uint8_t)gs;
    out[50] = 8;
    out[51] = (uint8_t)egs;
    put32(52, (uint32_t)sec.size());
    if (v2) {
      putf(84, 1.0f);  // embed_scale
      const uint16_t ne = (uint16_t)c.num_experts;
      std::memcpy(out + 105, &ne, 2);
      out[107] = (uint8_t)c.experts_per_token;
      out[108] = c.norm_topk_prob ? 1 : 0;
    }
    uint64_t off = hsz + sec.size() * 16;
    for (size_t i = 0; i < sec.size(); ++i) {
      const uint64_t sz = sec[i];
      std::memcpy(out + hsz + 16 * i, &off, 8);
      std::memcpy(out + hsz + 16 * i + 8, &sz, 8);
      off += sz;
    }
    uint8_t *w = out + hsz + sec.size() * 16;
    Lcg lcg{0x20260813ull};
    uint64_t tid = 0;
    std::vector<float> pre;  // the LCG mode's tensor, generated in file order
    auto source = [&](size_t rows, size_t cols) {
      Source s;
      if (c.mode == 2) {
        pre.resize(rows * cols);
        for (auto &x : pre) x = lcg.weight();
        s.pre = pre.data();
      } else {
        s.seed = seed;
        s.tid = ++tid;
        s.stdv = c.weight_std;
      }
      return s;
    };
    auto norm = [&](uint8_t *dst) {
      float *f = reinterpret_cast<float *>(dst);
      for (int i = 0; i < H; ++i) f[i] = c.mode == 2 ? lcg.norm() : 1.0f;
    };
    put_embedding(w, source(V, H), V, H, egs);
    w += sec[0];
    for (int l = 0; l < L; ++l) {
      for (int p = 0; p < 7; ++p) {
        put_linear(w, source(dims[p][0], dims[p][1]), dims[p][0], dims[p][1], gs, sym);
        w += linear_bytes(dims[p][0], dims[p][1], gs);
      }
      if (v2) {
        put_f32(w, source(c.num_experts, H), c.num_experts, H);
        w += (size_t)c.num_experts * H * 4;
        for (uint32_t e = 1; e < c.num_experts; ++e)
          for (int p = 4; p < 7; ++p) {
            put_linear(w, source(dims[p][0], dims[p][1]), dims[p][0], dims[p][1], gs, sym);
            w += linear_bytes(dims[p][0], dims[p][1], gs);
          }
      }
      norm(w);
      norm(w + (size_t)H * 4);
      w += 2 * (size_t)H * 4;
    }
    norm(w);
    w += (size_t)H * 4;
    if (!c.tied) {
      put_linear(w, source(V, H), V, H, gs, sym);
      w += linear_bytes(V, H, gs);
    }
    if ((size_t)(w - out) != total) fail(RAI_E_ARG, "synthetic image size mismatch");
  } catch (...) {
    std::free(img.data);
    throw;
  }
  return img;
}

}  // namespace rai

extern "C" int rai_synth_model(const rai_synth_config *cfg, uint64_t seed, const char *path,
                               uint8_t **image, size_t *image_len) {
  RAI_API_BODY({
    if (!cfg) rai::fail(RAI_E_ARG, "null config");
    if (!path && (!image || !image_len)) rai::fail(RAI_E_ARG, "image output pointers are null");
    rai::SynthImage img = rai::synth_model(*cfg, seed);
    if (path) {
      FILE *f = std::fopen(path, "wb");
      if (!f) {
        std::free(img.data);
        rai::fail(RAI_E_IO, std::string("cannot open ") + path);
      }
      const size_t n = std::fwrite(img.data, 1, img.size, f);
      const int rc = std::fclose(f);
      std::free(img.data);
      if (n != img.size || rc != 0) rai::fail(RAI_E_IO, std::string("short write to ") + path);
      if (image_len) *image_len = img.size;
    } else {
      *image = img.data;  // the caller frees it with rai_free_image
      *image_len = img.size;
    }
  });
}

extern "C" void rai_free_image(uint8_t *image) { std::free(image); }
