// Oracle: .raimodel reader, KV cache, forward passes and decoders, restated
// from rai-infer/src/{format,model,kv_cache,lookup,sampler}.rs.
// Test infrastructure only; see oracle.h.
#include <omp.h>

#include <cmath>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "ora_internal.h"
#include "oracle.h"

namespace ora {

static thread_local std::string g_err;
void set_error(const std::string &m) { g_err = m; }

struct Linear {
  int rows = 0, cols = 0, gs = 0;
  const uint8_t *params = nullptr;
  const uint8_t *nib = nullptr;
};

struct Layer {
  Linear lin[7];  // q k v o gate up down (format.rs:86-94 order)
  std::vector<Linear> experts;  // [e*3 + {0 gate,1 up,2 down}] for e in 0..E
  std::vector<float> router;    // [E * hidden]
  std::vector<float> in_norm, post_norm;
};

struct Model {
  std::vector<uint8_t> buf;
  ora_config cfg{};
  const uint8_t *emb_params = nullptr, *emb_codes = nullptr;
  std::vector<Layer> layers;
  std::vector<float> final_norm;
  Linear lm_head;
  bool tied = false;
  std::vector<float> rope_cos, rope_sin;
  float attn_scale = 0.0f;
};

struct KV {
  int layers = 0, nkv = 0, hd = 0, cap = 0;
  std::vector<std::vector<float>> k, v;  // per layer [nkv][cap][hd]
  std::vector<int> filled;
};

static uint32_t rd32(const uint8_t *p) {
  uint32_t v;
  std::memcpy(&v, p, 4);
  return v;
}
static uint64_t rd64(const uint8_t *p) {
  uint64_t v;
  std::memcpy(&v, p, 8);
  return v;
}
static float rdf(const uint8_t *p) {
  float v;
  std::memcpy(&v, p, 4);
  return v;
}

static void fail(const std::string &m) { throw std::runtime_error(m); }

static Linear read_linear(const uint8_t *base, size_t size, size_t &off, int rows, int cols,
                          int gs) {
  if (off + 8 > size) fail("linear header truncated");
  if ((int)rd32(base + off) != rows || (int)rd32(base + off + 4) != cols)
    fail("linear dimension mismatch");
  off += 8;
  const size_t groups = (cols + gs - 1) / gs;
  const size_t pbytes = (size_t)rows * groups * 4;
  const size_t nbytes = ((size_t)rows * cols + 1) / 2;
  if (off + pbytes + nbytes > size) fail("linear data truncated");
  Linear l;
  l.rows = rows;
  l.cols = cols;
  l.gs = gs;
  l.params = base + off;
  l.nib = base + off + pbytes;
  off += pbytes + nbytes;
  return l;
}

static std::vector<float> read_vec(const uint8_t *base, size_t size, size_t &off, size_t n) {
  if (off + n * 4 > size) fail("vector truncated");
  std::vector<float> v(n);
  std::memcpy(v.data(), base + off, n * 4);
  off += n * 4;
  return v;
}

// RaiModelFile::open + RaiModel::load (format.rs:557-1082, model.rs:97-181),
// restricted to the capability subset the oracle implements.
static void load(Model &m, int max_groups) {
  const uint8_t *d = m.buf.data();
  const size_t n = m.buf.size();
  if (n < 64 || std::memcmp(d, "RAIM", 4) != 0) fail("not a .raimodel file");
  ora_config &c = m.cfg;
  c.version = rd32(d + 4);
  if (c.version != 1 && c.version != 2) fail("unsupported version");
  const size_t hsz = c.version == 1 ? 64 : 128;
  if (n < hsz) fail("header truncated");
  c.hidden_size = rd32(d + 8);
  c.num_layers = rd32(d + 12);
  c.num_heads = rd32(d + 16);
  c.num_kv_heads = rd32(d + 20);
  c.head_dim = rd32(d + 24);
  c.intermediate_size = rd32(d + 28);
  c.vocab_size = rd32(d + 32);
  c.max_context = rd32(d + 36);
  c.rope_theta = rdf(d + 40);
  c.norm_eps = rdf(d + 44);
  if (d[48] != 4 || d[50] != 8) fail("unsupported bit widths");
  c.group_size = d[49];
  c.embed_group_size = d[51];
  c.embed_scale = 1.0f;
  c.attn_scale = 0.0f;
  if (c.version == 2) {
    if (d[64] != 0 || d[65] != 0 || d[66] != 0 || d[67] != 0) fail("unsupported v2 capability");
    for (int i = 68; i < 84; ++i)
      if (d[i]) fail("unsupported rope scaling");
    c.embed_scale = rdf(d + 84);
    if (rdf(d + 88) != 0.0f || rdf(d + 92) != 0.0f || rdf(d + 100) != 0.0f || d[104] != 0)
      fail("unsupported v2 capability");
    c.attn_scale = rdf(d + 96);
    uint16_t ne;
    std::memcpy(&ne, d + 105, 2);
    c.num_experts = ne;
    c.experts_per_token = d[107];
    c.norm_topk_prob = d[108] & 1;
  }
  const int H = c.hidden_size, F = c.intermediate_size, hd = c.head_dim;
  const int qd = c.num_heads * hd, kvd = c.num_kv_heads * hd, gs = c.group_size;
  if (gs == 0 || gs % 2 || c.embed_group_size == 0 || c.embed_group_size % 2) fail("bad group size");
  if (hd % 8 || c.num_heads % c.num_kv_heads) fail("bad attention shape");
  const int mg = std::max(std::max((H + gs - 1) / gs, (F + gs - 1) / gs), (qd + gs - 1) / gs);
  if (max_groups > 0 && mg > max_groups) fail("group count exceeds MAX_GROUPS");
  const uint32_t ns = rd32(d + 52);
  if (ns != c.num_layers + 2 && ns != c.num_layers + 3) fail("invalid section count");
  m.tied = ns == c.num_layers + 2;
  c.tied = m.tied;
  std::vector<std::pair<size_t, size_t>> sec(ns);
  size_t prev = hsz + (size_t)ns * 16;
  for (uint32_t i = 0; i < ns; ++i) {
    const size_t o = rd64(d + hsz + i * 16), s = rd64(d + hsz + i * 16 + 8);
    if (s == 0 || o != prev || o + s > n) fail("bad section table");
    sec[i] = {o, s};
    prev = o + s;
  }
  if (prev != n) fail("trailing data");
  // Section 0: embedding.
  {
    const size_t eg = (H + c.embed_group_size - 1) / c.embed_group_size;
    const size_t pb = (size_t)c.vocab_size * eg * 4;
    if (sec[0].second != pb + (size_t)c.vocab_size * H) fail("embedding size mismatch");
    m.emb_params = d + sec[0].first;
    m.emb_codes = d + sec[0].first + pb;
  }
  const int dims[7][2] = {{qd, H}, {kvd, H}, {kvd, H}, {H, qd}, {F, H}, {F, H}, {H, F}};
  m.layers.resize(c.num_layers);
  for (uint32_t li = 0; li < c.num_layers; ++li) {
    const uint8_t *b = d + sec[1 + li].first;
    const size_t sz = sec[1 + li].second;
    size_t off = 0;
    Layer &L = m.layers[li];
    for (int p = 0; p < 7; ++p) L.lin[p] = read_linear(b, sz, off, dims[p][0], dims[p][1], gs);
    if (c.num_experts > 0) {
      L.router = read_vec(b, sz, off, (size_t)c.num_experts * H);
      L.experts.resize((size_t)c.num_experts * 3);
      L.experts[0] = L.lin[4];
      L.experts[1] = L.lin[5];
      L.experts[2] = L.lin[6];
      for (uint32_t e = 1; e < c.num_experts; ++e)
        for (int p = 0; p < 3; ++p)
          L.experts[e * 3 + p] = read_linear(b, sz, off, dims[4 + p][0], dims[4 + p][1], gs);
    }
    L.in_norm = read_vec(b, sz, off, H);
    L.post_norm = read_vec(b, sz, off, H);
    if (off != sz) fail("layer section size mismatch");
  }
  {
    size_t off = 0;
    m.final_norm = read_vec(d + sec[1 + c.num_layers].first, sec[1 + c.num_layers].second, off, H);
    if (off != sec[1 + c.num_layers].second) fail("final norm size mismatch");
  }
  if (!m.tied) {
    size_t off = 0;
    const auto &s = sec[ns - 1];
    m.lm_head = read_linear(d + s.first, s.second, off, c.vocab_size, H, gs);
    if (off != s.second) fail("lm_head size mismatch");
  }
  rope_tables(m.rope_cos, m.rope_sin, hd, c.max_context, c.rope_theta);
  m.attn_scale = c.attn_scale > 0.0f ? c.attn_scale : 1.0f / std::sqrt((float)hd);
}

// KVCache (kv_cache.rs): f32 [kv_head][capacity][head_dim] per layer with a
// filled watermark.  Capacity is allocated up front (growth only re-strides,
// kv_cache.rs:105-126, and never changes a value).
static void kv_store(KV &kv, int layer, int pos, const float *k, const float *v) {
  if (pos >= kv.cap) fail("KV cache position is out of range");
  if (pos > kv.filled[layer]) fail("KV store would leave a gap");
  for (int h = 0; h < kv.nkv; ++h) {
    std::memcpy(&kv.k[layer][((size_t)h * kv.cap + pos) * kv.hd], k + h * kv.hd, kv.hd * 4);
    std::memcpy(&kv.v[layer][((size_t)h * kv.cap + pos) * kv.hd], v + h * kv.hd, kv.hd * 4);
  }
  kv.filled[layer] = std::max(kv.filled[layer], pos + 1);
}

static void attend(const Model &m, const KV &kv, int li, const float *q, int pos, float *out) {
  const ora_config &c = m.cfg;
  if (pos >= kv.filled[li]) fail("KV read at unwritten position");
  const int hpk = c.num_heads / c.num_kv_heads, hd = c.head_dim;
  std::vector<float> scores(pos + 1);
  for (uint32_t qh = 0; qh < c.num_heads; ++qh) {
    const int kvh = qh / hpk;
    attention_head(q + qh * hd, &kv.k[li][(size_t)kvh * kv.cap * hd],
                   &kv.v[li][(size_t)kvh * kv.cap * hd], pos, hd, m.attn_scale, out + qh * hd,
                   scores.data());
  }
}

// route_experts (layers.rs:1808-1870): router logits (dot_f32, a
// sequential f32 sum), softmax over all experts, top-k by selection sort
// (ties: lowest index), optional renormalisation of the chosen weights.
static void route_experts(const float *router, const float *x, int H, int E, int topk, bool norm_topk,
                          std::vector<int> &sel, std::vector<float> &wts) {
  std::vector<float> probs(E);
  for (int e = 0; e < E; ++e) {
    float s = -0.0f;  // Rust's f32 Sum starts at -0.0
    for (int i = 0; i < H; ++i) s += router[(size_t)e * H + i] * x[i];
    probs[e] = s;
  }
  float mx = -INFINITY;
  for (float p : probs) mx = std::fmax(mx, p);
  float sum = 0.0f;
  for (float &p : probs) {
    p = std::exp(p - mx);
    sum += p;
  }
  for (float &p : probs) p /= sum;
  sel.clear();
  wts.clear();
  std::vector<bool> taken(E, false);
  for (int k = 0; k < topk; ++k) {
    int best = -1;
    float bv = -INFINITY;
    for (int e = 0; e < E; ++e)
      if (!taken[e] && probs[e] > bv) {
        bv = probs[e];
        best = e;
      }
    if (best < 0) break;
    taken[best] = true;
    sel.push_back(best);
    wts.push_back(bv);
  }
  if (norm_topk) {
    float tot = -0.0f;
    for (float w : wts) tot += w;
    if (tot > 0.0f)
      for (float &w : wts) w /= tot;
  }
}

// The MoE arm of mlp_block (model.rs:208-261) for one token.
static void moe_token(const Model &m, const Layer &L, const float *x, float *out) {
  const ora_config &c = m.cfg;
  const int H = c.hidden_size, F = c.intermediate_size, E = c.num_experts;
  std::vector<int> sel;
  std::vector<float> wts;
  route_experts(L.router.data(), x, H, E, (int)c.experts_per_token, c.norm_topk_prob != 0, sel, wts);
  std::vector<float> gate(F), up(F), eo(H);
  for (int i = 0; i < H; ++i) out[i] = 0.0f;
  for (size_t s = 0; s < sel.size(); ++s) {
    const Linear *ex = &L.experts[(size_t)sel[s] * 3];
    matmul(gate.data(), ex[0].nib, ex[0].params, x, F, H, 1, ex[0].gs);
    matmul(up.data(), ex[1].nib, ex[1].params, x, F, H, 1, ex[1].gs);
    silu_mul(gate.data(), up.data(), F);
    matmul(eo.data(), ex[2].nib, ex[2].params, gate.data(), H, F, 1, ex[2].gs);
    for (int i = 0; i < H; ++i) out[i] += wts[s] * eo[i];
  }
}

static void lin(const Linear &l, const float *x, float *out, int batch) {
  matmul(out, l.nib, l.params, x, l.rows, l.cols, batch, l.gs);
}

// RaiModel::forward_batch (model.rs:692-963).  With batch == 1 this is also
// forward_from_hidden (model.rs:407-499): fused QKV / gate-up share one
// quantization, which is the same per-projection arithmetic, and the
// reference states (and tests, model_invariants.rs:92-134) the two agree.
static void forward(const Model &m, KV &kv, float *hid, const int *positions, int batch) {
  const ora_config &c = m.cfg;
  const int H = c.hidden_size, F = c.intermediate_size, hd = c.head_dim;
  const int qd = c.num_heads * hd, kvd = c.num_kv_heads * hd;
  for (int b = 0; b < batch; ++b) {
    if (positions[b] >= (int)c.max_context) fail("batch position exceeds model context");
    if (b > 0 && positions[b] != positions[b - 1] + 1) fail("batch positions must be consecutive");
  }
  std::vector<float> normed((size_t)batch * H), resid((size_t)batch * H);
  std::vector<float> qb((size_t)batch * qd), kb((size_t)batch * kvd), vb((size_t)batch * kvd);
  std::vector<float> att((size_t)batch * qd), ob((size_t)batch * H);
  std::vector<float> gb((size_t)batch * F), ub((size_t)batch * F), mo((size_t)batch * H);
  const int half = hd / 2;
  for (uint32_t li = 0; li < c.num_layers; ++li) {
    const Layer &L = m.layers[li];
    for (int b = 0; b < batch; ++b)
      rms_norm_residual(&normed[(size_t)b * H], &resid[(size_t)b * H], hid + (size_t)b * H,
                        L.in_norm.data(), H, c.norm_eps);
    lin(L.lin[0], normed.data(), qb.data(), batch);
    lin(L.lin[1], normed.data(), kb.data(), batch);
    lin(L.lin[2], normed.data(), vb.data(), batch);
    for (int b = 0; b < batch; ++b) {
      const int p = positions[b];
      rope_apply(&qb[(size_t)b * qd], c.num_heads, hd, &m.rope_cos[(size_t)p * half],
                 &m.rope_sin[(size_t)p * half]);
      rope_apply(&kb[(size_t)b * kvd], c.num_kv_heads, hd, &m.rope_cos[(size_t)p * half],
                 &m.rope_sin[(size_t)p * half]);
      kv_store(kv, li, p, &kb[(size_t)b * kvd], &vb[(size_t)b * kvd]);
    }
    std::string err;
#pragma omp parallel for schedule(dynamic)
    for (int b = 0; b < batch; ++b) {
      try {
        attend(m, kv, li, &qb[(size_t)b * qd], positions[b], &att[(size_t)b * qd]);
      } catch (const std::exception &e) {
#pragma omp critical
        err = e.what();
      }
    }
    if (!err.empty()) fail(err);
    lin(L.lin[3], att.data(), ob.data(), batch);
    for (int b = 0; b < batch; ++b)
      vec_add(hid + (size_t)b * H, &resid[(size_t)b * H], &ob[(size_t)b * H], H);
    for (int b = 0; b < batch; ++b)
      rms_norm_residual(&normed[(size_t)b * H], &resid[(size_t)b * H], hid + (size_t)b * H,
                        L.post_norm.data(), H, c.norm_eps);
    if (c.num_experts > 0) {
      for (int b = 0; b < batch; ++b) moe_token(m, L, &normed[(size_t)b * H], &mo[(size_t)b * H]);
    } else {
      lin(L.lin[4], normed.data(), gb.data(), batch);
      lin(L.lin[5], normed.data(), ub.data(), batch);
      for (int b = 0; b < batch; ++b) silu_mul(&gb[(size_t)b * F], &ub[(size_t)b * F], F);
      lin(L.lin[6], gb.data(), mo.data(), batch);
    }
    for (int b = 0; b < batch; ++b)
      vec_add(hid + (size_t)b * H, &resid[(size_t)b * H], &mo[(size_t)b * H], H);
  }
}

// hidden_to_logits_batch (model.rs:966-1033) / hidden_to_logits_into.
static void logits(const Model &m, const float *hid, float *out, int batch) {
  const ora_config &c = m.cfg;
  const int H = c.hidden_size, V = c.vocab_size;
  std::vector<float> normed((size_t)batch * H);
  for (int b = 0; b < batch; ++b)
    rms_norm(&normed[(size_t)b * H], hid + (size_t)b * H, m.final_norm.data(), H, c.norm_eps);
  if (!m.tied) {
    lin(m.lm_head, normed.data(), out, batch);
  } else {
    for (int b = 0; b < batch; ++b)
      tied_lm_head(out + (size_t)b * V, &normed[(size_t)b * H], m.emb_codes, m.emb_params, V, H,
                   c.embed_group_size);
  }
}

// embed_token (model.rs:371-403).
static void embed(const Model &m, int tok, float *out) {
  const ora_config &c = m.cfg;
  if (tok < 0 || tok >= (int)c.vocab_size) fail("token id is out of model vocabulary");
  embed_lookup(out, tok, m.emb_codes, m.emb_params, c.hidden_size, c.embed_group_size);
  if (c.embed_scale != 1.0f)
    for (uint32_t i = 0; i < c.hidden_size; ++i) out[i] *= c.embed_scale;
}

// find_ngram_draft (lookup.rs:131-171).
static bool find_ngram(const int32_t *t, int64_t len, int64_t mn, int64_t mx, int64_t maxd,
                       int64_t *res) {
  if (maxd == 0 || len < 2) return false;
  const int64_t hi = std::min(mx, len - 1);
  const int64_t lo = std::max<int64_t>(mn, 1);
  if (lo > hi) return false;
  for (int64_t n = hi; n >= lo; --n) {
    const int32_t *suf = t + len - n;
    for (int64_t s = len - n - 1; s >= 0; --s) {
      if (std::memcmp(t + s, suf, n * sizeof(int32_t)) != 0) continue;
      const int64_t ds = s + n;
      const int64_t dl = std::min(maxd, len - ds);
      if (dl == 0) continue;
      res[0] = n;
      res[1] = ds;
      res[2] = dl;
      return true;
    }
  }
  return false;
}

struct Lookup {
  const Model *m;
  KV kv;
  int max_ctx;
};

}  // namespace ora

using namespace ora;

struct ora_model {
  Model m;
};
struct ora_kv {
  KV kv;
};
struct ora_lookup {
  Lookup d;
};


static KV make_kv(const Model &m, int max_ctx) {
  const ora_config &c = m.cfg;
  if (max_ctx <= 0) fail("KV cache context must be non-zero");
  KV kv;
  kv.layers = c.num_layers;
  kv.nkv = c.num_kv_heads;
  kv.hd = c.head_dim;
  kv.cap = std::min<int>(max_ctx, c.max_context);
  kv.k.resize(kv.layers);
  kv.v.resize(kv.layers);
  for (int l = 0; l < kv.layers; ++l) {
    kv.k[l].assign((size_t)kv.nkv * kv.cap * kv.hd, 0.0f);
    kv.v[l].assign((size_t)kv.nkv * kv.cap * kv.hd, 0.0f);
  }
  kv.filled.assign(kv.layers, 0);
  return kv;
}

extern "C" {

void ora_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }
int ora_get_threads(void) { return omp_get_max_threads(); }
const char *ora_last_error(void) { return ora::g_err.c_str(); }

int ora_quantize_split(const float *x, int cols, int gs, int8_t *qe, int8_t *qo, float *sc) {
  ORA_TRY(quantize_split(x, cols, gs, qe, qo, sc));
}
int ora_input_sums(const float *x, int cols, int gs, float *sums) {
  ORA_TRY(input_sums(x, cols, gs, sums));
}
int ora_w4a8_matvec(float *out, const uint8_t *nib, const uint8_t *params, const float *x,
                    int rows, int cols, int gs) {
  ORA_TRY(matmul(out, nib, params, x, rows, cols, 1, gs));
}
int ora_w4a8_matmul(float *out, const uint8_t *nib, const uint8_t *params, const float *x,
                    int rows, int cols, int m, int gs) {
  ORA_TRY(matmul(out, nib, params, x, rows, cols, m, gs));
}
static void all_lane_sums(int32_t *out, const uint8_t *nib, const float *x, int rows, int cols,
                          int m, int gs) {
  const int groups = (cols + gs - 1) / gs;
  for (int t = 0; t < m; ++t) {
    QuantInput q = quantize_token(x + (size_t)t * cols, cols, gs);
#pragma omp parallel for
    for (int r = 0; r < rows; ++r)
      lane_sums(nib + (size_t)r * (cols / 2), q, cols, gs,
                out + ((size_t)t * rows + r) * groups * 12);
  }
}

int ora_w4a8_lane_sums(int32_t *out, const uint8_t *nib, const float *x, int rows, int cols,
                       int m, int gs) {
  ORA_TRY(all_lane_sums(out, nib, x, rows, cols, m, gs));
}
int ora_tied_lm_head(float *logits, const float *hidden, const uint8_t *codes,
                     const uint8_t *params, int vocab, int n, int gs) {
  ORA_TRY(tied_lm_head(logits, hidden, codes, params, vocab, n, gs));
}
int ora_embed_lookup(float *out, int token, const uint8_t *codes, const uint8_t *params,
                     int vocab, int n, int gs) {
  ORA_TRY({
    if (token < 0 || token >= vocab) fail("token id is out of range");
    embed_lookup(out, token, codes, params, n, gs);
  });
}
int ora_rms_norm(float *out, const float *x, const float *w, int n, float eps) {
  ORA_TRY(rms_norm(out, x, w, n, eps));
}
int ora_rms_norm_residual(float *normed, float *resid, const float *x, const float *w, int n,
                          float eps) {
  ORA_TRY(rms_norm_residual(normed, resid, x, w, n, eps));
}
int ora_silu_mul(float *gate, const float *up, int n) { ORA_TRY(silu_mul(gate, up, n)); }
int ora_rope_tables(float *cos_t, float *sin_t, int hd, int max_ctx, float theta) {
  ORA_TRY({
    std::vector<float> c, s;
    rope_tables(c, s, hd, max_ctx, theta);
    std::memcpy(cos_t, c.data(), c.size() * 4);
    std::memcpy(sin_t, s.data(), s.size() * 4);
  });
}
int ora_rope_apply(float *heads, int nh, int hd, const float *c, const float *s) {
  ORA_TRY(rope_apply(heads, nh, hd, c, s));
}
int ora_attention_head(const float *q, const float *k, const float *v, int pos, int hd,
                       float scale, float *out) {
  ORA_TRY({
    std::vector<float> sc(pos + 1);
    attention_head(q, k, v, pos, hd, scale, out, sc.data());
  });
}
float ora_expf(float x) { return std::exp(x); }
float ora_schraudolph(float x) { return schraudolph(x); }

int64_t ora_argmax(const float *v, int64_t n) { return argmax(v, n); }
int ora_find_ngram_draft(const int32_t *t, int64_t len, int64_t mn, int64_t mx, int64_t maxd,
                         int64_t *res) {
  return find_ngram(t, len, mn, mx, maxd, res) ? 1 : 0;
}

int ora_model_open(const uint8_t *buf, size_t len, int max_groups, ora_model **out) {
  ORA_TRY({
    auto p = std::make_unique<ora_model>();
    p->m.buf.assign(buf, buf + len);
    load(p->m, max_groups);
    *out = p.release();
  });
}
void ora_model_free(ora_model *m) { delete m; }
int ora_model_config(const ora_model *m, ora_config *out) { ORA_TRY(*out = m->m.cfg); }
int ora_kv_create(const ora_model *m, int max_ctx, ora_kv **out) {
  ORA_TRY({
    auto p = std::make_unique<ora_kv>();
    p->kv = make_kv(m->m, max_ctx);
    *out = p.release();
  });
}
void ora_kv_free(ora_kv *kv) { delete kv; }
int ora_kv_truncate(ora_kv *kv, int len) {
  ORA_TRY(for (int &f : kv->kv.filled) f = std::min(f, len));
}
int ora_kv_filled(const ora_kv *kv, int layer) { return kv->kv.filled.at(layer); }
int ora_kv_read(const ora_kv *kv, int layer, int head, int pos, int which, float *out) {
  ORA_TRY({
    const KV &k = kv->kv;
    if (layer < 0 || layer >= k.layers || head < 0 || head >= k.nkv) fail("KV head out of range");
    if (pos < 0 || pos >= k.filled[layer]) fail("KV read above the watermark");
    const std::vector<float> &src = which == 0 ? k.k[layer] : k.v[layer];
    std::memcpy(out, &src[((size_t)head * k.cap + pos) * k.hd], sizeof(float) * k.hd);
  });
}
int ora_route_experts(const float *router, const float *x, int hidden, int num_experts, int topk,
                      int norm_topk_prob, int32_t *experts, float *weights) {
  ORA_TRY({
    std::vector<int> sel;
    std::vector<float> wts;
    route_experts(router, x, hidden, num_experts, topk, norm_topk_prob != 0, sel, wts);
    for (int k = 0; k < topk; ++k) {
      experts[k] = k < (int)sel.size() ? sel[k] : -1;
      weights[k] = k < (int)wts.size() ? wts[k] : 0.0f;
    }
  });
}
int ora_embed_token(const ora_model *m, int token, float *out) { ORA_TRY(embed(m->m, token, out)); }
int ora_forward_from_hidden(const ora_model *m, ora_kv *kv, float *hidden, int pos, int store_kv) {
  ORA_TRY({
    if (!store_kv) fail("probe passes (store_kv = false) are not part of the lookup path");
    forward(m->m, kv->kv, hidden, &pos, 1);
  });
}
int ora_forward_batch(const ora_model *m, ora_kv *kv, float *hiddens, const int32_t *positions,
                      int batch) {
  ORA_TRY({
    if (batch <= 0) fail("batch must contain at least one token");
    forward(m->m, kv->kv, hiddens, positions, batch);
  });
}
int ora_hidden_to_logits(const ora_model *m, const float *hidden, float *out) {
  ORA_TRY(logits(m->m, hidden, out, 1));
}
int ora_hidden_to_logits_batch(const ora_model *m, const float *hiddens, float *out, int batch) {
  ORA_TRY(logits(m->m, hiddens, out, batch));
}

int ora_lookup_create(const ora_model *m, int max_ctx, ora_lookup **out) {
  ORA_TRY({
    auto p = std::make_unique<ora_lookup>();
    p->d.m = &m->m;
    p->d.max_ctx = std::min<int>(max_ctx, m->m.cfg.max_context);
    if (p->d.max_ctx <= 0) fail("prompt-lookup context must be non-zero");
    p->d.kv = make_kv(m->m, p->d.max_ctx);
    *out = p.release();
  });
}
void ora_lookup_free(ora_lookup *d) { delete d; }
// KVCache::store (kv_cache.rs:143-173) for positions 0..npos of one layer at
// once: rows [kv_head][npos][head_dim] of K (which = 0) or V (1); the
// layer's watermark becomes npos.
static void import_rows(KV &k, int layer, int which, const float *rows, int npos) {
  if (layer < 0 || layer >= k.layers) fail("layer out of range");
  if (npos < 0 || npos > k.cap) fail("positions exceed the cache");
  std::vector<float> &dst = which == 0 ? k.k[layer] : k.v[layer];
  for (int h = 0; h < k.nkv; ++h)
    std::memcpy(&dst[(size_t)h * k.cap * k.hd], rows + (size_t)h * npos * k.hd, sizeof(float) * npos * k.hd);
  k.filled[layer] = npos;
}
int ora_kv_import(ora_kv *kv, int layer, int which, const float *rows, int npos) {
  ORA_TRY(import_rows(kv->kv, layer, which, rows, npos));
}
int ora_lookup_import_kv(ora_lookup *dd, int layer, int which, const float *rows, int npos) {
  ORA_TRY(import_rows(dd->d.kv, layer, which, rows, npos));
}
int ora_lookup_kv_filled(const ora_lookup *d) { return d->d.kv.filled.at(0); }

// The plain sampled step of the `rai run` loop without speculation
// (run.rs:692-735): decode_one's forward of `token` at `pos`, then the
// repetition penalty over ctx[0..len) and sample_token with the whole
// SamplerConfig (sampler.rs:47-199), drawing from `rng`.
int ora_lookup_decode_sample(ora_lookup *dd, int pos, int token, const int32_t *ctx, int len, float temperature,
                             int64_t top_k, float top_p, float penalty, ora_rng *rng, int32_t *out) {
  ORA_TRY({
    Lookup &d = dd->d;
    const Model &m = *d.m;
    const int H = m.cfg.hidden_size, V = m.cfg.vocab_size;
    if (pos < 0 || pos >= d.max_ctx) fail("decode position exceeds the context window");
    if (token < 0 || token >= V) fail("token id is out of model vocabulary");
    std::vector<float> h(H), lg(V);
    embed(m, token, h.data());
    forward(m, d.kv, h.data(), &pos, 1);
    logits(m, h.data(), lg.data(), 1);
    int tok = 0;
    if (ora_sample_plain(lg.data(), V, ctx, len, temperature, top_k, top_p, penalty, rng, &tok))
      fail("sample_token failed");
    *out = tok;
  });
}

// decode_one (lookup.rs:428-455) with argmax: the plain greedy step of the
// `rai run` loop without speculation.
int ora_lookup_decode_one(ora_lookup *dd, int pos, int token, int32_t *out) {
  ORA_TRY({
    Lookup &d = dd->d;
    const Model &m = *d.m;
    const int H = m.cfg.hidden_size, V = m.cfg.vocab_size;
    if (pos < 0 || pos >= d.max_ctx) fail("decode position exceeds the context window");
    if (token < 0 || token >= V) fail("token id is out of model vocabulary");
    std::vector<float> h(H), lg(V);
    embed(m, token, h.data());
    forward(m, d.kv, h.data(), &pos, 1);
    logits(m, h.data(), lg.data(), 1);
    *out = (int32_t)argmax(lg.data(), V);
  });
}

// LookupDecoder::prefill (lookup.rs:219-247).
int ora_lookup_prefill(ora_lookup *dd, const int32_t *prompt, int n, int *pos_out) {
  ORA_TRY({
    Lookup &d = dd->d;
    const int H = d.m->cfg.hidden_size;
    if (n <= 0) fail("prompt must contain at least one token");
    if (n > d.max_ctx) fail("prompt exceeds the prompt-lookup context window");
    const int cnt = n - 1;
    if (cnt > 0) {
      std::vector<float> h((size_t)cnt * H);
      std::vector<int> pos(cnt);
      for (int i = 0; i < cnt; ++i) {
        embed(*d.m, prompt[i], &h[(size_t)i * H]);
        pos[i] = i;
      }
      forward(*d.m, d.kv, h.data(), pos.data(), cnt);
    }
    *pos_out = cnt;
  });
}

// LookupDecoder::step (lookup.rs:260-425) with greedy acceptance: accept
// while argmax(logits_i) == draft_i, emit argmax at the first mismatch, emit
// the bonus argmax when every draft token is accepted.
int ora_lookup_step_greedy(ora_lookup *dd, int pos, const int32_t *ctx, int len, int max_draft,
                           int min_ngram, int max_ngram, int32_t *out, ora_metrics *met) {
  ORA_TRY({
    Lookup &d = dd->d;
    const Model &m = *d.m;
    const int H = m.cfg.hidden_size, V = m.cfg.vocab_size;
    if (max_draft <= 0 || min_ngram < 1 || min_ngram > max_ngram) fail("invalid lookup config");
    if (len <= 0) fail("prompt-lookup step requires a non-empty context");
    if (pos >= d.max_ctx) fail("decode position exceeds the context window");
    const int last = ctx[len - 1];
    const int budget = std::max(0, d.max_ctx - pos - 1);
    int64_t mt[3] = {0, 0, 0};
    const bool hit = budget > 0 && find_ngram(ctx, len, min_ngram, max_ngram,
                                              std::min(max_draft, budget), mt);
    if (!hit) {
      // decode_one (lookup.rs:428-455)
      std::vector<float> h(H), lg(V);
      embed(m, last, h.data());
      forward(m, d.kv, h.data(), &pos, 1);
      logits(m, h.data(), lg.data(), 1);
      out[0] = (int32_t)argmax(lg.data(), V);
      *met = {0, 0, 1, 0};
      return 0;
    }
    const int nd = (int)mt[2];
    for (int i = 0; i < nd; ++i)
      if (ctx[mt[1] + i] < 0 || ctx[mt[1] + i] >= V)
        fail("context contains a token outside the model vocabulary");
    const int vb = nd + 1;
    std::vector<float> h((size_t)vb * H), lg((size_t)vb * V);
    std::vector<int> ps(vb);
    for (int i = 0; i < vb; ++i) {
      embed(m, i == 0 ? last : ctx[mt[1] + i - 1], &h[(size_t)i * H]);
      ps[i] = pos + i;
    }
    forward(m, d.kv, h.data(), ps.data(), vb);
    logits(m, h.data(), lg.data(), vb);
    int acc = 0, prod = 0;
    for (int i = 0; i < nd; ++i) {
      const int a = (int)argmax(&lg[(size_t)i * V], V);
      out[prod++] = a;
      if (a != ctx[mt[1] + i]) break;
      ++acc;
    }
    if (acc == nd) out[prod++] = (int32_t)argmax(&lg[(size_t)nd * V], V);
    for (int &f : d.kv.filled) f = std::min(f, pos + prod);
    *met = {acc, nd, prod, (int32_t)mt[0]};
  });
}

// LookupDecoder::step (lookup.rs:260-425) with exact sampling at
// `temperature` (> 1e-6): the verify forward as in the greedy step, then the
// accept / correct / bonus loop of lookup.rs:359-403 drawing from `rng`;
// decode_one samples its token (lookup.rs:428-455).
int ora_lookup_step_sampled(ora_lookup *dd, int pos, const int32_t *ctx, int len, int max_draft,
                            int min_ngram, int max_ngram, float temperature, ora_rng *rng, int32_t *out,
                            ora_metrics *met) {
  ORA_TRY({
    Lookup &d = dd->d;
    const Model &m = *d.m;
    const int H = m.cfg.hidden_size, V = m.cfg.vocab_size;
    if (max_draft <= 0 || min_ngram < 1 || min_ngram > max_ngram) fail("invalid lookup config");
    if (!(std::isfinite(temperature) && temperature > 1e-6f)) fail("exact sampling needs temperature > 1e-6");
    if (len <= 0) fail("prompt-lookup step requires a non-empty context");
    if (pos >= d.max_ctx) fail("decode position exceeds the context window");
    const int last = ctx[len - 1];
    const int budget = std::max(0, d.max_ctx - pos - 1);
    int64_t mt[3] = {0, 0, 0};
    const bool hit = budget > 0 && find_ngram(ctx, len, min_ngram, max_ngram,
                                              std::min(max_draft, budget), mt);
    if (!hit) {
      std::vector<float> h(H), lg(V);
      embed(m, last, h.data());
      forward(m, d.kv, h.data(), &pos, 1);
      logits(m, h.data(), lg.data(), 1);
      int tok = 0;
      if (ora_sample_token(lg.data(), V, temperature, rng, &tok)) fail("sample_token failed");
      out[0] = tok;
      *met = {0, 0, 1, 0};
      return 0;
    }
    const int nd = (int)mt[2];
    for (int i = 0; i < nd; ++i)
      if (ctx[mt[1] + i] < 0 || ctx[mt[1] + i] >= V)
        fail("context contains a token outside the model vocabulary");
    const int vb = nd + 1;
    std::vector<float> h((size_t)vb * H), lg((size_t)vb * V);
    std::vector<int> ps(vb);
    for (int i = 0; i < vb; ++i) {
      embed(m, i == 0 ? last : ctx[mt[1] + i - 1], &h[(size_t)i * H]);
      ps[i] = pos + i;
    }
    forward(m, d.kv, h.data(), ps.data(), vb);
    logits(m, h.data(), lg.data(), vb);
    int prod = 0, acc = 0;
    if (ora_sampled_accept(lg.data(), V, ctx + mt[1], nd, temperature, rng, out, &prod, &acc))
      fail("sampled acceptance failed");
    for (int &f : d.kv.filled) f = std::min(f, pos + prod);
    *met = {acc, nd, prod, (int32_t)mt[0]};
  });
}

// SpeculativeDecoder (speculative.rs:79-391): a draft model proposes k
// tokens one decode step at a time, the target verifies [last, drafts] in
// one batched forward, then exact acceptance (temperature > 1e-6) or, below
// that, greedy acceptance (draft tokens by argmax, accepted while the
// target's argmax agrees).
struct ora_spec {
  const Model *draft, *target;
  KV dkv, tkv;
  int max_ctx;
};

int ora_spec_create(const ora_model *draft, const ora_model *target, int max_ctx, ora_spec **out) {
  ORA_TRY({
    if (draft->m.cfg.vocab_size != target->m.cfg.vocab_size) fail("draft and target vocabularies differ");
    const int dctx = std::min(max_ctx, (int)draft->m.cfg.max_context);
    const int tctx = std::min(max_ctx, (int)target->m.cfg.max_context);
    const int ctx = std::min(dctx, tctx);
    if (ctx <= 0) fail("speculative decoding context must be non-zero");
    auto d = new ora_spec{&draft->m, &target->m, make_kv(draft->m, dctx), make_kv(target->m, tctx), ctx};
    *out = d;
  });
}
void ora_spec_free(ora_spec *d) { delete d; }

int ora_spec_prefill(ora_spec *d, const int32_t *prompt, int n, int *pos_out) {
  ORA_TRY({
    if (n <= 0) fail("prompt must contain at least one token");
    if (n > d->max_ctx) fail("prompt exceeds the speculative context window");
    const int cnt = n - 1;
    for (int w = 0; w < 2; ++w) {
      const Model &m = w ? *d->target : *d->draft;
      KV &kv = w ? d->tkv : d->dkv;
      const int H = m.cfg.hidden_size;
      for (int p = 0; p < cnt; ++p) {
        std::vector<float> h(H);
        embed(m, prompt[p], h.data());
        forward(m, kv, h.data(), &p, 1);
      }
    }
    *pos_out = cnt;
  });
}

int ora_spec_step(ora_spec *d, int pos, int last, int draft_k, float temperature, ora_rng *rng, int32_t *out,
                  ora_metrics *met) {
  ORA_TRY({
    const Model &dm = *d->draft, &tm = *d->target;
    const int V = tm.cfg.vocab_size, DH = dm.cfg.hidden_size, TH = tm.cfg.hidden_size;
    const bool sampled = std::isfinite(temperature) && temperature > 1e-6f;
    if (draft_k <= 0) fail("speculative draft_k must be non-zero");
    if (pos >= d->max_ctx) fail("decode position exceeds the speculative context window");
    const int k = std::min(draft_k, std::max(0, d->max_ctx - pos - 1));
    auto pick = [&](std::vector<float> &lg) {
      int t = 0;
      if (!sampled) return (int)argmax(lg.data(), V);
      if (ora_sample_token(lg.data(), V, temperature, rng, &t)) fail("sample_token failed");
      return t;
    };
    if (k == 0) {
      std::vector<float> h(TH), lg(V);
      embed(tm, last, h.data());
      forward(tm, d->tkv, h.data(), &pos, 1);
      logits(tm, h.data(), lg.data(), 1);
      out[0] = pick(lg);
      *met = {0, 0, 1, 0};
      return 0;
    }
    std::vector<int32_t> toks(k + 1);
    std::vector<float> dl((size_t)k * V);
    toks[0] = last;
    for (int i = 0; i < k; ++i) {
      std::vector<float> h(DH), lg(V);
      embed(dm, toks[i], h.data());
      int p = pos + i;
      forward(dm, d->dkv, h.data(), &p, 1);
      logits(dm, h.data(), lg.data(), 1);
      std::copy(lg.begin(), lg.end(), dl.begin() + (size_t)i * V);
      toks[i + 1] = pick(lg);
    }
    std::vector<float> h((size_t)(k + 1) * TH), tl((size_t)(k + 1) * V);
    std::vector<int> ps(k + 1);
    for (int i = 0; i <= k; ++i) {
      embed(tm, toks[i], &h[(size_t)i * TH]);
      ps[i] = pos + i;
    }
    forward(tm, d->tkv, h.data(), ps.data(), k + 1);
    logits(tm, h.data(), tl.data(), k + 1);
    int acc = 0, prod = 0;
    if (sampled) {
      if (ora_spec_accept(tl.data(), dl.data(), V, toks.data() + 1, k, temperature, rng, out, &prod, &acc))
        fail("speculative acceptance failed");
    } else {
      for (int i = 0; i < k; ++i) {
        const int a = (int)argmax(&tl[(size_t)i * V], V);
        out[prod++] = a;
        if (a != toks[i + 1]) break;
        ++acc;
      }
      if (acc == k) out[prod++] = (int32_t)argmax(&tl[(size_t)k * V], V);
    }
    if (acc == k) {
      // The last draft token has not been through the draft model yet.
      std::vector<float> hd(DH);
      embed(dm, toks[k], hd.data());
      int p = pos + k;
      forward(dm, d->dkv, hd.data(), &p, 1);
    }
    for (int &f : d->dkv.filled) f = std::min(f, pos + prod);
    for (int &f : d->tkv.filled) f = std::min(f, pos + prod);
    *met = {acc, k, prod, 0};
  });
}

int ora_greedy_generate(const ora_model *mm, const int32_t *prompt, int n, int steps, int max_ctx,
                        int32_t *out) {
  ORA_TRY({
    const Model &m = mm->m;
    const int H = m.cfg.hidden_size, V = m.cfg.vocab_size;
    if (n <= 0) fail("prompt must contain at least one token");
    if (n + steps > max_ctx + 1) fail("generation exceeds the context window");
    KV kv = make_kv(m, max_ctx);
    const int cnt = n - 1;
    if (cnt > 0) {
      std::vector<float> h((size_t)cnt * H);
      std::vector<int> pos(cnt);
      for (int i = 0; i < cnt; ++i) {
        embed(m, prompt[i], &h[(size_t)i * H]);
        pos[i] = i;
      }
      forward(m, kv, h.data(), pos.data(), cnt);
    }
    int last = prompt[n - 1];
    std::vector<float> h(H), lg(V);
    for (int s = 0; s < steps; ++s) {
      const int pos = cnt + s;
      embed(m, last, h.data());
      forward(m, kv, h.data(), &pos, 1);
      logits(m, h.data(), lg.data(), 1);
      last = (int)argmax(lg.data(), V);
      out[s] = last;
    }
  });
}

}  // extern "C"
