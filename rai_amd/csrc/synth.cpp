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

struct Writer {
  std::vector<uint8_t> buf;
  void u32(uint32_t v) { raw(&v, 4); }
  void f32(float v) { raw(&v, 4); }
  void u16(uint16_t v) { raw(&v, 2); }
  void raw(const void *p, size_t n) {
    const uint8_t *b = (const uint8_t *)p;
    buf.insert(buf.end(), b, b + n);
  }
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

// Quantize one [rows][cols] weight matrix and append it as a linear
// ([u32 rows][u32 cols][params][nibbles], raimodel.py:518-526).
void put_linear(Writer &w, const std::vector<float> &wt, int rows, int cols, int gs, bool sym) {
  const int groups = (cols + gs - 1) / gs;
  std::vector<uint16_t> params((size_t)rows * groups * 2);
  std::vector<uint8_t> codes((size_t)rows * cols);
  auto work = [&](int r0, int r1) {
    for (int r = r0; r < r1; ++r) {
      const float *row = &wt[(size_t)r * cols];
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
            codes[(size_t)r * cols + c] = (uint8_t)((int)q + 8);
          }
        } else {
          minmax_params(row + c0, c1 - c0, 16, s16, z16, s64, z64);
          for (int c = c0; c < c1; ++c) {
            const double q = std::min(15.0, std::max(0.0, std::nearbyint(((double)row[c] - z64) / s64)));
            codes[(size_t)r * cols + c] = (uint8_t)q;
          }
        }
        params[((size_t)r * groups + g) * 2] = s16;
        params[((size_t)r * groups + g) * 2 + 1] = z16;
      }
    }
  };
  const int nt = std::max(1, std::min<int>((int)std::thread::hardware_concurrency(), 16));
  std::vector<std::thread> th;
  for (int i = 0; i < nt; ++i) th.emplace_back(work, rows * i / nt, rows * (i + 1) / nt);
  for (auto &t : th) t.join();
  w.u32(rows);
  w.u32(cols);
  w.raw(params.data(), params.size() * 2);
  const size_t base = w.buf.size();
  w.buf.resize(base + (size_t)rows * cols / 2);
  for (size_t i = 0; i < (size_t)rows * cols / 2; ++i)
    w.buf[base + i] = (uint8_t)((codes[2 * i] & 0x0F) | ((codes[2 * i + 1] & 0x0F) << 4));
}

void put_embedding(Writer &w, const std::vector<float> &wt, int vocab, int hidden, int egs) {
  const int groups = (hidden + egs - 1) / egs;
  std::vector<uint16_t> params((size_t)vocab * groups * 2);
  std::vector<uint8_t> codes((size_t)vocab * hidden);
  for (int v = 0; v < vocab; ++v)
    for (int g = 0; g < groups; ++g) {
      const int c0 = g * egs, c1 = std::min(hidden, c0 + egs);
      uint16_t s16, z16;
      double s64, z64;
      minmax_params(&wt[(size_t)v * hidden + c0], c1 - c0, 256, s16, z16, s64, z64);
      params[((size_t)v * groups + g) * 2] = s16;
      params[((size_t)v * groups + g) * 2 + 1] = z16;
      for (int c = c0; c < c1; ++c) {
        const double q = std::min(
            255.0, std::max(0.0, std::nearbyint(((double)wt[(size_t)v * hidden + c] - z64) / s64)));
        codes[(size_t)v * hidden + c] = (uint8_t)q;
      }
    }
  w.raw(params.data(), params.size() * 2);
  w.raw(codes.data(), codes.size());
}

}  // namespace

std::vector<uint8_t> synth_model(const rai_synth_config &c, uint64_t seed) {
  if (c.mode > 2) fail(RAI_E_ARG, "unknown synth mode");
  if (c.num_experts != 0 && c.mode == 2) fail(RAI_E_ARG, "the LCG fixture mode is dense only");
  const int H = c.hidden_size, F = c.intermediate_size, V = c.vocab_size, L = c.num_layers;
  const int qd = c.num_heads * c.head_dim, kvd = c.num_kv_heads * c.head_dim;
  const int gs = c.group_size, egs = c.embed_group_size;
  if (H <= 0 || F <= 0 || V <= 0 || L <= 0 || gs <= 0 || egs <= 0 || c.num_kv_heads == 0)
    fail(RAI_E_ARG, "invalid synthetic model shape");
  const bool sym = c.mode == 0;
  const bool v2 = c.num_experts > 0;
  Lcg lcg{0x20260813ull};
  uint64_t tid = 0;
  auto tensor = [&](size_t rows, size_t cols, bool is_norm = false) {
    std::vector<float> t(rows * cols);
    if (c.mode == 2) {
      for (auto &x : t) x = is_norm ? lcg.norm() : lcg.weight();
    } else if (is_norm) {
      std::fill(t.begin(), t.end(), 1.0f);
    } else {
      const uint64_t id = ++tid;
      const size_t n = t.size();
      const int nt = std::max(1, std::min<int>((int)std::thread::hardware_concurrency(), 16));
      std::vector<std::thread> th;
      for (int i = 0; i < nt; ++i)
        th.emplace_back([&, i] {
          for (size_t j = n * i / nt; j < n * (i + 1) / nt; ++j) t[j] = gauss(seed, id, j, c.weight_std);
        });
      for (auto &x : th) x.join();
    }
    return t;
  };
  std::vector<std::vector<uint8_t>> sections;
  {
    Writer w;
    put_embedding(w, tensor(V, H), V, H, egs);
    sections.push_back(std::move(w.buf));
  }
  const int dims[7][2] = {{qd, H}, {kvd, H}, {kvd, H}, {H, qd}, {F, H}, {F, H}, {H, F}};
  for (int l = 0; l < L; ++l) {
    Writer w;
    for (int p = 0; p < 7; ++p) put_linear(w, tensor(dims[p][0], dims[p][1]), dims[p][0], dims[p][1], gs, sym);
    if (v2) {
      std::vector<float> router = tensor(c.num_experts, H);
      w.raw(router.data(), router.size() * 4);
      for (uint32_t e = 1; e < c.num_experts; ++e)
        for (int p = 4; p < 7; ++p)
          put_linear(w, tensor(dims[p][0], dims[p][1]), dims[p][0], dims[p][1], gs, sym);
    }
    std::vector<float> n1 = tensor(1, H, true), n2 = tensor(1, H, true);
    w.raw(n1.data(), H * 4);
    w.raw(n2.data(), H * 4);
    sections.push_back(std::move(w.buf));
  }
  {
    std::vector<float> fn = tensor(1, H, true);
    Writer w;
    w.raw(fn.data(), H * 4);
    sections.push_back(std::move(w.buf));
  }
  if (!c.tied) {
    Writer w;
    put_linear(w, tensor(V, H), V, H, gs, sym);
    sections.push_back(std::move(w.buf));
  }
  // Header (raimodel.py:558-579; v2 capability block per format.rs:21-40).
  Writer out;
  const size_t hsz = v2 ? 128 : 64;
  out.buf.assign(hsz, 0);
  std::memcpy(out.buf.data(), "RAIM", 4);
  auto put32 = [&](size_t off, uint32_t v) { std::memcpy(out.buf.data() + off, &v, 4); };
  auto putf = [&](size_t off, float v) { std::memcpy(out.buf.data() + off, &v, 4); };
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
  out.buf[48] = 4;
  out.buf[49] = (uint8_t)gs;
  out.buf[50] = 8;
  out.buf[51] = (uint8_t)egs;
  put32(52, (uint32_t)sections.size());
  if (v2) {
    putf(84, 1.0f);  // embed_scale
    const uint16_t ne = (uint16_t)c.num_experts;
    std::memcpy(out.buf.data() + 105, &ne, 2);
    out.buf[107] = (uint8_t)c.experts_per_token;
    out.buf[108] = c.norm_topk_prob ? 1 : 0;
  }
  uint64_t off = hsz + sections.size() * 16;
  for (auto &s : sections) {
    const uint64_t sz = s.size();
    out.raw(&off, 8);
    out.raw(&sz, 8);
    off += sz;
  }
  size_t total = out.buf.size();
  for (auto &s : sections) total += s.size();
  out.buf.reserve(total);
  for (auto &s : sections) {
    out.raw(s.data(), s.size());
    std::vector<uint8_t>().swap(s);
  }
  return std::move(out.buf);
}

}  // namespace rai

extern "C" int rai_synth_model(const rai_synth_config *cfg, uint64_t seed, const char *path,
                               uint8_t **image, size_t *image_len) {
  RAI_API_BODY({
    if (!cfg) rai::fail(RAI_E_ARG, "null config");
    std::vector<uint8_t> img = rai::synth_model(*cfg, seed);
    if (path) {
      FILE *f = std::fopen(path, "wb");
      if (!f) rai::fail(RAI_E_IO, std::string("cannot open ") + path);
      const size_t n = std::fwrite(img.data(), 1, img.size(), f);
      const int rc = std::fclose(f);
      if (n != img.size() || rc != 0) rai::fail(RAI_E_IO, std::string("short write to ") + path);
      if (image_len) *image_len = img.size();
    } else {
      if (!image || !image_len) rai::fail(RAI_E_ARG, "image output pointers are null");
      uint8_t *p = (uint8_t *)std::malloc(img.size());
      if (!p) rai::fail(RAI_E_OOM, "image allocation failed");
      std::memcpy(p, img.data(), img.size());
      *image = p;
      *image_len = img.size();
    }
  });
}

extern "C" void rai_free_image(uint8_t *image) { std::free(image); }
