// Host runtime and C ABI: device model, KV cache, forward passes, the
// prompt-lookup decoder.  Mirrors rai-infer/src/{model,kv_cache,lookup}.rs.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "common.h"
#include "format.h"
#include "kernels.h"

namespace rai {

static thread_local std::string g_last_error;
void set_last_error(const std::string &m) { g_last_error = m; }

#define HIP_CHECK(expr)                                                                  \
  do {                                                                                   \
    hipError_t e_ = (expr);                                                              \
    if (e_ != hipSuccess)                                                                \
      fail(e_ == hipErrorOutOfMemory ? RAI_E_OOM : RAI_E_HIP,                            \
           std::string(#expr) + ": " + hipGetErrorString(e_));                           \
  } while (0)

// Tokens per forward chunk (prefill is split into chunks of this size; the
// per-token arithmetic does not depend on the split).
constexpr int kChunk = 1024;

struct DevBuf {
  void *p = nullptr;
  DevBuf() = default;
  DevBuf(const DevBuf &) = delete;
  DevBuf &operator=(const DevBuf &) = delete;
  ~DevBuf() {
    if (p) (void)hipFree(p);
  }
  void alloc(size_t n) {
    if (p) (void)hipFree(p);
    p = nullptr;
    if (n == 0) n = 256;
    HIP_CHECK(hipMalloc(&p, n));
  }
  template <class T>
  T *as() const {
    return reinterpret_cast<T *>(p);
  }
};

struct DLinear {
  int rows = 0, cols = 0, gs = 0;
  const uint8_t *nib = nullptr, *params = nullptr;
  // The parameters again in 16-row tiles (launch_params_tile16), read by
  // the matrix-core GEMV of 2..64 tokens; null where that does not apply.
  const uint8_t *params_tiled = nullptr;
};

struct DLayer {
  DLinear lin[7];
  // q|k|v and gate|up stored back to back (same cols): one GEMV each.
  // rows == 0 when the pieces could not be placed contiguously.
  DLinear qkv, gate_up;
  std::vector<DLinear> experts;  // all experts, 3 linears each (expert 0 = lin[4..6])
  bool experts_gu = false;       // every expert's gate and up placed back to back
  const float *router = nullptr;
  const float *in_norm = nullptr, *post_norm = nullptr;
};

struct Workspace;

}  // namespace rai

using namespace rai;

struct rai_model {
  rai_model_config cfg{};
  ModelView view;
  DevBuf arena;
  std::vector<DLayer> layers;
  const uint8_t *emb_params = nullptr, *emb_codes = nullptr;
  const float *final_norm = nullptr;
  DLinear lm_head;
  bool tied = false;
  const float *rope_cos = nullptr, *rope_sin = nullptr;
  float attn_scale = 1.0f;
  uint64_t weight_bytes = 0;
  hipStream_t stream = nullptr;
  std::unique_ptr<Workspace> ws;  // for the model-level host-buffer API
  // Sparse layers: per layer 6 * num_experts device pointers, the code and
  // parameter arrays of gate|up (expert-major, gate then up), then of down.
  DevBuf moe_tab;
  DevBuf tiled;  // the params_tiled copies
  ~rai_model();
};

struct rai_kv {
  rai_model *model = nullptr;
  int layers = 0, nkv = 0, hd = 0;
  size_t cap = 0;
  size_t vstride = 0;  // cap rounded up to 64: the d-major V row length
  DevBuf k, v;         // K [layer][nkv][cap][hd]; V d-major [layer][nkv][hd][vstride]
  std::vector<size_t> filled;
  float *kc(int l) const { return k.as<float>() + (size_t)l * nkv * cap * hd; }
  float *vc(int l) const { return v.as<float>() + (size_t)l * nkv * hd * vstride; }
  size_t k_bytes() const { return (size_t)layers * nkv * cap * hd * sizeof(float); }
  size_t v_bytes() const { return (size_t)layers * nkv * hd * vstride * sizeof(float); }
};

namespace rai {

// Per-context scratch for up to `maxm` tokens.
struct Workspace {
  int maxm = 0;
  DevBuf hid, normed, qb, kb, vb, att, ob, gb, ub, mo, logits, am;
  DevBuf qkvb, gub;  // fused q|k|v and gate|up outputs [m][rows]
  DevBuf q_nat, q_split, qscale, qsum, hq;
  DevBuf qa;   // activations packed for the matrix-core W4A8 kernel (<= 64 tokens)
  DevBuf qmm;  // activation records of the matrix-core W4A8 GEMM (> 64 tokens)
  DevBuf err;
  // Attention score/probability rows; grown to the largest KV capacity seen.
  DevBuf scores;
  size_t scores_n = 0;
  float *attn_scores(const rai_model_config &c, size_t cap) {
    const size_t n = attention_scores_floats(maxm, (int)c.num_heads, (int)cap);
    if (n > scores_n) {
      scores.alloc(n * sizeof(float));
      scores_n = n;
    }
    return scores.as<float>();
  }
  // MoE
  DevBuf sel, wts, eo, xg, yg, gg, ug, idx, wcol;
  // Device MoE path: entry plan, gathered quantized inputs, gate|up outputs.
  DevBuf moff, ment_of, ment_tok, ment_exp, mq, msc, msu, mgu, mlogit;
  int logit_rows = 0;
  void init(const rai_model &m, int maxm_, int logit_rows_) {
    const rai_model_config &c = m.cfg;
    maxm = maxm_;
    logit_rows = logit_rows_;
    const size_t H = c.hidden_size, F = c.intermediate_size, qd = (size_t)c.num_heads * c.head_dim;
    const size_t kvd = (size_t)c.num_kv_heads * c.head_dim, V = c.vocab_size;
    const size_t K = std::max(std::max(H, F), qd);
    const size_t G = ceil_div(K, std::min(c.group_size, c.embed_group_size)) + 1;
    auto f = [&](DevBuf &b, size_t n) { b.alloc(n * sizeof(float) * maxm); };
    f(hid, H);
    f(normed, H);
    f(qb, qd);
    f(kb, kvd);
    f(vb, kvd);
    f(att, qd);
    f(ob, H);
    f(gb, F);
    f(ub, F);
    f(mo, H);
    f(qkvb, qd + 2 * kvd);
    f(gub, 2 * F);
    logits.alloc(sizeof(float) * V * std::max(1, logit_rows));
    am.alloc(sizeof(uint32_t) * maxm);
    q_nat.alloc(K * maxm);
    q_split.alloc(K * maxm);
    qa.alloc(sizeof(_Float16) * qa_pack_halves(std::min(maxm, kMfmaMaxTokens), (int)K));
    if (maxm > kMfmaMaxTokens) qmm.alloc(mm_pack_bytes(maxm, (int)K));
    hq.alloc(H * maxm);
    qscale.alloc(sizeof(float) * G * maxm);
    qsum.alloc(sizeof(float) * G * maxm);
    err.alloc(sizeof(int) * 4);
    HIP_CHECK(hipMemset(err.p, 0, sizeof(int) * 4));
    if (c.num_experts > 0) {
      sel.alloc(sizeof(int) * maxm * c.experts_per_token);
      wts.alloc(sizeof(float) * maxm * c.experts_per_token);
      eo.alloc(sizeof(float) * maxm * c.experts_per_token * H);
      xg.alloc(sizeof(float) * maxm * H);
      yg.alloc(sizeof(float) * maxm * H);
      gg.alloc(sizeof(float) * maxm * F);
      ug.alloc(sizeof(float) * maxm * F);
      idx.alloc(sizeof(int) * maxm * c.experts_per_token);
      const size_t ne = (size_t)maxm * c.experts_per_token;
      moff.alloc(sizeof(int) * (c.num_experts + 1));
      ment_of.alloc(sizeof(int) * ne);
      ment_tok.alloc(sizeof(int) * ne);
      ment_exp.alloc(sizeof(int) * ne);
      mq.alloc(ne * std::max(H, F));
      msc.alloc(sizeof(float) * ne * G);
      msu.alloc(sizeof(float) * ne * G);
      mgu.alloc(sizeof(float) * ne * 2 * F);
      mlogit.alloc(sizeof(float) * maxm * c.num_experts);
      wcol.alloc(sizeof(float) * maxm);
    }
  }
};

}  // namespace rai

rai_model::~rai_model() {
  ws.reset();
  if (stream) (void)hipStreamDestroy(stream);
}

namespace rai {

// ------------------------------------------------------------- loading --

static void upload_model(rai_model &m, const uint8_t *img, size_t len, int max_groups) {
  m.view = parse_model(img, len, max_groups);
  const ModelView &v = m.view;
  m.cfg = v.cfg;
  m.tied = v.tied;
  m.attn_scale = v.attention_scale;
  const rai_model_config &c = m.cfg;
  if (c.max_context == 0) fail(RAI_E_FORMAT, "max_context is zero");
  // Arena layout: every piece 256-byte aligned, in the reference's byte layout.
  struct Piece {
    size_t src, len, dst;
  };
  std::vector<Piece> pieces;
  size_t total = 0;
  auto add = [&](size_t src, size_t n) {
    total = (total + 255) & ~size_t(255);
    pieces.push_back({src, n, total});
    total += n;
    return pieces.size() - 1;
  };
  const size_t H = c.hidden_size;
  const size_t eg = ceil_div(H, c.embed_group_size);
  const size_t pe = add(v.emb_params_off, (size_t)c.vocab_size * eg * 4);
  const size_t ce = add(v.emb_codes_off, (size_t)c.vocab_size * H);
  struct LinIdx {
    size_t p, n;
  };
  std::vector<std::vector<LinIdx>> lidx(c.num_layers);
  std::vector<size_t> router_idx(c.num_layers), n1_idx(c.num_layers), n2_idx(c.num_layers);
  uint64_t wbytes = 0;
  for (uint32_t l = 0; l < c.num_layers; ++l) {
    const LayerView &L = v.layers[l];
    // q, k, v and gate, up: codes back to back, then params back to back,
    // so each set can run as one matrix.
    size_t ni[7], pi[7];
    for (int p : {0, 1, 2}) ni[p] = add(L.lin[p].nib_off, L.lin[p].nib_len);
    for (int p : {0, 1, 2}) pi[p] = add(L.lin[p].params_off, L.lin[p].params_len);
    pi[3] = add(L.lin[3].params_off, L.lin[3].params_len);
    ni[3] = add(L.lin[3].nib_off, L.lin[3].nib_len);
    for (int p : {4, 5}) ni[p] = add(L.lin[p].nib_off, L.lin[p].nib_len);
    for (int p : {4, 5}) pi[p] = add(L.lin[p].params_off, L.lin[p].params_len);
    pi[6] = add(L.lin[6].params_off, L.lin[6].params_len);
    ni[6] = add(L.lin[6].nib_off, L.lin[6].nib_len);
    for (int p = 0; p < 7; ++p) {
      lidx[l].push_back({pi[p], ni[p]});
      wbytes += L.lin[p].params_len + L.lin[p].nib_len;
    }
    // Experts past the first (whose gate|up are lin[4], lin[5] above): gate
    // and up codes back to back, then their params back to back, then down,
    // so each expert's gate|up runs as one matrix of 2F rows.
    for (size_t e = 0; e + 2 < L.experts.size(); e += 3) {
      const LinearView &g = L.experts[e], &u = L.experts[e + 1], &d = L.experts[e + 2];
      const size_t gn = add(g.nib_off, g.nib_len), un = add(u.nib_off, u.nib_len);
      const size_t gp = add(g.params_off, g.params_len), up = add(u.params_off, u.params_len);
      const size_t dp = add(d.params_off, d.params_len), dn = add(d.nib_off, d.nib_len);
      lidx[l].push_back({gp, gn});
      lidx[l].push_back({up, un});
      lidx[l].push_back({dp, dn});
    }
    if (c.num_experts > 0) router_idx[l] = add(L.router_off, (size_t)c.num_experts * H * 4);
    n1_idx[l] = add(L.in_norm_off, H * 4);
    n2_idx[l] = add(L.post_norm_off, H * 4);
  }
  const size_t fn = add(v.final_norm_off, H * 4);
  size_t lmp = 0, lmn = 0;
  if (!m.tied) {
    lmp = add(v.lm_head.params_off, v.lm_head.params_len);
    lmn = add(v.lm_head.nib_off, v.lm_head.nib_len);
    wbytes += v.lm_head.params_len + v.lm_head.nib_len;
  } else {
    wbytes += (size_t)c.vocab_size * (H + eg * 4);
  }
  // RoPE tables: RoPETable::with_scaling (layers.rs:561-633) on the host with
  // the C library's powf/cosf/sinf, exactly as the reference computes them.
  const size_t half = c.head_dim / 2;
  std::vector<float> cosv((size_t)c.max_context * half), sinv((size_t)c.max_context * half);
  {
    std::vector<float> inv(half);
    for (size_t i = 0; i < half; ++i)
      inv[i] = 1.0f / std::pow(c.rope_theta, (2.0f * (float)i) / (float)c.head_dim);
    for (size_t p = 0; p < c.max_context; ++p)
      for (size_t i = 0; i < half; ++i) {
        const float ang = (float)p * inv[i];
        cosv[p * half + i] = std::cos(ang);
        sinv[p * half + i] = std::sin(ang);
      }
  }
  total = (total + 255) & ~size_t(255);
  const size_t rope_off = total;
  total += 2 * cosv.size() * sizeof(float) + 256;
  m.arena.alloc(total);
  uint8_t *base = m.arena.as<uint8_t>();
  // Stage through a pinned buffer in 64 MiB slices.
  const size_t slice = 64ull << 20;
  uint8_t *pin = nullptr;
  HIP_CHECK(hipHostMalloc((void **)&pin, slice, hipHostMallocDefault));
  try {
    for (const Piece &pc : pieces) {
      for (size_t o = 0; o < pc.len; o += slice) {
        const size_t n = std::min(slice, pc.len - o);
        std::memcpy(pin, img + pc.src + o, n);
        HIP_CHECK(hipMemcpy(base + pc.dst + o, pin, n, hipMemcpyHostToDevice));
      }
    }
  } catch (...) {
    (void)hipHostFree(pin);
    throw;
  }
  HIP_CHECK(hipHostFree(pin));
  HIP_CHECK(hipMemcpy(base + rope_off, cosv.data(), cosv.size() * 4, hipMemcpyHostToDevice));
  HIP_CHECK(hipMemcpy(base + rope_off + cosv.size() * 4, sinv.data(), sinv.size() * 4,
                      hipMemcpyHostToDevice));
  m.rope_cos = reinterpret_cast<const float *>(base + rope_off);
  m.rope_sin = reinterpret_cast<const float *>(base + rope_off + cosv.size() * 4);
  m.emb_params = base + pieces[pe].dst;
  m.emb_codes = base + pieces[ce].dst;
  const int qd = c.num_heads * c.head_dim, kvd = c.num_kv_heads * c.head_dim;
  const int dims[7][2] = {{qd, (int)H}, {kvd, (int)H}, {kvd, (int)H}, {(int)H, qd},
                          {(int)c.intermediate_size, (int)H}, {(int)c.intermediate_size, (int)H},
                          {(int)H, (int)c.intermediate_size}};
  m.layers.resize(c.num_layers);
  for (uint32_t l = 0; l < c.num_layers; ++l) {
    DLayer &D = m.layers[l];
    auto mk = [&](size_t k, int p) {
      DLinear d;
      d.rows = dims[p][0];
      d.cols = dims[p][1];
      d.gs = c.group_size;
      d.params = base + pieces[lidx[l][k].p].dst;
      d.nib = base + pieces[lidx[l][k].n].dst;
      return d;
    };
    for (int p = 0; p < 7; ++p) D.lin[p] = mk(p, p);
    auto contiguous = [&](std::initializer_list<int> ps) {
      int prev = -1;
      for (int p : ps) {
        if (prev >= 0) {
          const Piece &a = pieces[lidx[l][prev].n], &b = pieces[lidx[l][p].n];
          const Piece &pa = pieces[lidx[l][prev].p], &pb = pieces[lidx[l][p].p];
          if (a.dst + a.len != b.dst || pa.dst + pa.len != pb.dst) return false;
        }
        prev = p;
      }
      return true;
    };
    if (contiguous({0, 1, 2})) {
      D.qkv = D.lin[0];
      D.qkv.rows = D.lin[0].rows + D.lin[1].rows + D.lin[2].rows;
    }
    if (c.num_experts == 0 && contiguous({4, 5})) {
      D.gate_up = D.lin[4];
      D.gate_up.rows = D.lin[4].rows + D.lin[5].rows;
    }
    if (c.num_experts > 0) {
      D.experts.push_back(D.lin[4]);
      D.experts.push_back(D.lin[5]);
      D.experts.push_back(D.lin[6]);
      for (size_t k = 7; k < lidx[l].size(); ++k) D.experts.push_back(mk(k, 4 + (int)((k - 7) % 3)));
      // Every expert's gate and up back to back (codes and params): one
      // gate|up matrix per expert for the entry GEMV.
      bool gu = contiguous({4, 5});
      for (int e = 1; e < (int)c.num_experts && gu; ++e) gu = contiguous({4 + 3 * e, 5 + 3 * e});
      D.experts_gu = gu;
      D.router = reinterpret_cast<const float *>(base + pieces[router_idx[l]].dst);
      // Expert bytes a decode step streams: experts_per_token of them.
      wbytes += (uint64_t)(c.experts_per_token - 1) *
                (v.layers[l].lin[4].params_len + v.layers[l].lin[4].nib_len +
                 v.layers[l].lin[5].params_len + v.layers[l].lin[5].nib_len +
                 v.layers[l].lin[6].params_len + v.layers[l].lin[6].nib_len);
    }
    D.in_norm = reinterpret_cast<const float *>(base + pieces[n1_idx[l]].dst);
    D.post_norm = reinterpret_cast<const float *>(base + pieces[n2_idx[l]].dst);
  }
  m.final_norm = reinterpret_cast<const float *>(base + pieces[fn].dst);
  if (!m.tied) {
    m.lm_head.rows = c.vocab_size;
    m.lm_head.cols = H;
    m.lm_head.gs = c.group_size;
    m.lm_head.params = base + pieces[lmp].dst;
    m.lm_head.nib = base + pieces[lmn].dst;
  }
  m.weight_bytes = wbytes;
  if (c.num_experts > 0) {
    const size_t E = c.num_experts;
    std::vector<const uint8_t *> tab(6 * E * c.num_layers);
    for (uint32_t l = 0; l < c.num_layers; ++l) {
      const DLayer &D = m.layers[l];
      const uint8_t **t = tab.data() + 6 * E * l;
      for (size_t e = 0; e < E; ++e) {
        for (int j = 0; j < 2; ++j) {
          t[2 * e + j] = D.experts[3 * e + j].nib;
          t[2 * E + 2 * e + j] = D.experts[3 * e + j].params;
        }
        t[4 * E + e] = D.experts[3 * e + 2].nib;
        t[5 * E + e] = D.experts[3 * e + 2].params;
      }
    }
    m.moe_tab.alloc(sizeof(void *) * tab.size());
    HIP_CHECK(hipMemcpy(m.moe_tab.p, tab.data(), sizeof(void *) * tab.size(), hipMemcpyHostToDevice));
  }
  HIP_CHECK(hipStreamCreateWithFlags(&m.stream, hipStreamNonBlocking));
  // Tile-layout copies of the parameters of the matrices the batched
  // forward runs through the matrix-core GEMV (about a fifth of the weight
  // bytes again; decode reads only the originals).
  {
    std::vector<DLinear *> tl;
    for (DLayer &D : m.layers) {
      if (D.qkv.rows) tl.push_back(&D.qkv);
      else for (int p : {0, 1, 2}) tl.push_back(&D.lin[p]);
      tl.push_back(&D.lin[3]);
      if (c.num_experts == 0) {
        if (D.gate_up.rows) tl.push_back(&D.gate_up);
        else for (int p : {4, 5}) tl.push_back(&D.lin[p]);
        tl.push_back(&D.lin[6]);
      }
    }
    if (!m.tied) tl.push_back(&m.lm_head);
    size_t tb = 0;
    for (DLinear *L : tl)
      if (params_tile16_ok(L->rows, L->cols, L->gs)) tb += ((size_t)L->rows * (L->cols / 32) * 4 + 255) & ~size_t(255);
    if (tb) {
      m.tiled.alloc(tb);
      uint8_t *p = m.tiled.as<uint8_t>();
      for (DLinear *L : tl) {
        if (!params_tile16_ok(L->rows, L->cols, L->gs)) continue;
        launch_params_tile16(L->params, L->rows, L->cols, p, m.stream);
        L->params_tiled = p;
        p += ((size_t)L->rows * (L->cols / 32) * 4 + 255) & ~size_t(255);
      }
      HIP_CHECK(hipGetLastError());
      HIP_CHECK(hipStreamSynchronize(m.stream));
    }
  }
}

// ------------------------------------------------------------- forward --

static void linear(const DLinear &L, const float *x, const Workspace &w, float *out, int m,
                   hipStream_t s, const float *add = nullptr) {
  launch_w4a8(out, add, L.nib, L.params, x, w.q_nat.as<int8_t>(), w.q_split.as<int8_t>(),
              w.qscale.as<float>(), w.qsum.as<float>(), L.rows, L.cols, m, L.gs, s,
              w.qa.as<_Float16>(), w.qmm.as<uint8_t>(), L.params_tiled);
}

// After any quantization of m rows of k columns into the workspace: pack
// the activations for the matrix-core kernel when it applies.
static void pack_for_mfma(const rai_model &md, int m, int k, const Workspace &w, hipStream_t s) {
  if (w4a8_mfma_path(1, k, m, md.cfg.group_size))
    launch_qa_pack(w.q_split.as<int8_t>(), m, k, w.qa.as<_Float16>(), s);
}

// The matrix-core activation buffer for a fused quantizer to fill directly
// (null when the matrix-core GEMV does not apply).
static _Float16 *mfma_acts(const rai_model &md, int m, int k, const Workspace &w) {
  return w4a8_mfma_path(1, k, m, md.cfg.group_size) ? w.qa.as<_Float16>() : nullptr;
}

static void quantize(const rai_model &md, const float *x, int m, int k, const Workspace &w,
                     hipStream_t s) {
  if (fused_quant_ok(k, md.cfg.group_size)) {
    launch_quant(x, m, k, md.cfg.group_size, w.q_split.as<int8_t>(), nullptr, w.qscale.as<float>(),
                 w.qsum.as<float>(), s, mfma_acts(md, m, k, w));
  } else {
    launch_quantize(x, m, k, md.cfg.group_size, w.q_nat.as<int8_t>(), w.q_split.as<int8_t>(),
                    w.qscale.as<float>(), w.qsum.as<float>(), s);
    pack_for_mfma(md, m, k, w, s);
  }
}

// The MLP of a sparse layer: mlp_block's MoE arm (model.rs:208-261) for
// every token, grouping each expert's tokens into one GEMV batch (each
// token's arithmetic is the M = 1 arithmetic: matmul == matvec).
static bool moe_on_device(const rai_model &md) {
  const rai_model_config &c = md.cfg;
  return md.moe_tab.p && moe_device_path((int)c.hidden_size, (int)c.intermediate_size, (int)c.group_size,
                                         (int)c.num_experts) &&
         fused_quant_ok((int)c.intermediate_size, (int)c.group_size);
}

// The sparse MLP with every step on the device (no host synchronisation);
// w.q_split / qscale / qsum hold the quantized normalised rows.  Adds the
// block's output to the hidden states (model.rs:208-261, then the residual).
static void moe_block_device(const rai_model &md, int li, Workspace &w, int m, hipStream_t s) {
  const rai_model_config &c = md.cfg;
  const DLayer &L = md.layers[li];
  const int H = c.hidden_size, F = c.intermediate_size, E = c.num_experts, K = c.experts_per_token;
  const int gs = c.group_size, ne = m * K;
  const uint8_t *const *tab = md.moe_tab.as<const uint8_t *>() + (size_t)6 * E * li;
  launch_router(w.normed.as<float>(), L.router, m, H, E, K, c.norm_topk_prob, w.sel.as<int>(),
                w.wts.as<float>(), w.mlogit.as<float>(), s);
  // Entry GEMVs: every expert's gate|up one matrix, entry t * K + k (slot k
  // of token t) through the one-token kernel, the token's quantized row read
  // in place; no plan: each block reads its entry's expert from the router's
  // picks, and the combine walks the slots in order.
  if (L.experts_gu && w4a8_dec_path(2 * F, H, gs) && w4a8_dec_path(H, F, gs)) {
    DecMoe gu{tab, tab + 2 * E, 2, w.sel.as<int>(), K, true, E, 2 * F};
    const DecMoe dn{tab + 4 * E, tab + 5 * E, 1, w.sel.as<int>(), K, false, E, H};
    gu.qo = w.mq.as<int8_t>();
    gu.so = w.msc.as<float>();
    gu.uo = w.msu.as<float>();
    // gate|up with silu_mul and the quantization of the entry rows fused,
    // else the two steps apart.
    bool done = launch_w4a8_dec_moe_glu(gu, w.q_split.as<int8_t>(), w.qscale.as<float>(), w.qsum.as<float>(),
                                        2 * F, H, gs, ne, s);
    if (!done && launch_w4a8_dec_moe(w.mgu.as<float>(), gu, w.q_split.as<int8_t>(), w.qscale.as<float>(),
                                     w.qsum.as<float>(), 2 * F, H, gs, ne, s)) {
      launch_silu_quant(w.mgu.as<float>(), w.mgu.as<float>() + F, ne, F, 2 * F, gs, w.mq.as<int8_t>(), nullptr,
                        w.msc.as<float>(), w.msu.as<float>(), s, nullptr);
      done = true;
    }
    if (done) {
      if (!launch_w4a8_dec_moe(w.eo.as<float>(), dn, w.mq.as<int8_t>(), w.msc.as<float>(), w.msu.as<float>(), H,
                               F, gs, ne, s))
        fail(RAI_E_UNSUPPORTED, "expert down projection shape");
      launch_moe_combine_sel(w.hid.as<float>(), w.eo.as<float>(), w.wts.as<float>(), w.sel.as<int>(), m, K, H, s);
      return;
    }
  }
  launch_moe_plan(w.sel.as<int>(), m, K, E, w.moff.as<int>(), w.ment_of.as<int>(), w.ment_tok.as<int>(),
                  w.ment_exp.as<int>(), s);
  launch_moe_gather(w.q_split.as<int8_t>(), w.qscale.as<float>(), w.qsum.as<float>(), w.ment_tok.as<int>(),
                    w.moff.as<int>(), E, ne, H, H / gs, w.mq.as<int8_t>(), w.msc.as<float>(), w.msu.as<float>(), s);
  launch_moe_gemv(w.mgu.as<float>(), 2 * F, tab, tab + 2 * E, 2, F, H, gs, E, w.mq.as<int8_t>(), w.msc.as<float>(),
                  w.msu.as<float>(), w.moff.as<int>(), s);
  launch_silu_quant(w.mgu.as<float>(), w.mgu.as<float>() + F, ne, F, 2 * F, gs, w.mq.as<int8_t>(), nullptr,
                    w.msc.as<float>(), w.msu.as<float>(), s, nullptr);
  launch_moe_gemv(w.eo.as<float>(), H, tab + 4 * E, tab + 5 * E, 1, H, F, gs, E, w.mq.as<int8_t>(),
                  w.msc.as<float>(), w.msu.as<float>(), w.moff.as<int>(), s);
  launch_moe_combine(w.hid.as<float>(), w.eo.as<float>(), w.wts.as<float>(), w.ment_of.as<int>(), m, K, H, s);
}

// Prefill-sized batches (more than kMfmaMaxTokens tokens): the same plan
// and gather, then the per-expert offsets on the host (one synchronisation
// per layer) and each expert's rows through the regular W4A8 kernels, which
// are far faster than the grouped one once an expert holds many rows.
static void moe_block_device_large(const rai_model &md, int li, Workspace &w, int m, hipStream_t s) {
  const rai_model_config &c = md.cfg;
  const DLayer &L = md.layers[li];
  const int H = c.hidden_size, F = c.intermediate_size, E = c.num_experts, K = c.experts_per_token;
  const int gs = c.group_size, ne = m * K, G = H / gs, GF = F / gs;
  launch_router(w.normed.as<float>(), L.router, m, H, E, K, c.norm_topk_prob, w.sel.as<int>(),
                w.wts.as<float>(), w.mlogit.as<float>(), s);
  launch_moe_plan(w.sel.as<int>(), m, K, E, w.moff.as<int>(), w.ment_of.as<int>(), w.ment_tok.as<int>(), nullptr,
                  s);
  launch_moe_gather(w.q_split.as<int8_t>(), w.qscale.as<float>(), w.qsum.as<float>(), w.ment_tok.as<int>(),
                    w.moff.as<int>(), E, ne, H, G, w.mq.as<int8_t>(), w.msc.as<float>(), w.msu.as<float>(), s);
  std::vector<int> off(E + 1);
  HIP_CHECK(hipMemcpyAsync(off.data(), w.moff.p, sizeof(int) * (E + 1), hipMemcpyDeviceToHost, s));
  HIP_CHECK(hipStreamSynchronize(s));
  float *gate = w.mgu.as<float>(), *up = gate + (size_t)ne * F;
  auto run = [&](const DLinear &lin, const int8_t *q, const float *sc, const float *su, int groups, int o, int cnt,
                 float *out) {
    const _Float16 *qa = nullptr;
    if (w4a8_mfma_path(lin.rows, lin.cols, cnt, lin.gs)) {
      launch_qa_pack(q + (size_t)o * lin.cols, cnt, lin.cols, w.qa.as<_Float16>(), s);
      qa = w.qa.as<_Float16>();
    }
    launch_w4a8(out, nullptr, lin.nib, lin.params, nullptr, nullptr, q + (size_t)o * lin.cols,
                sc + (size_t)o * groups, su + (size_t)o * groups, lin.rows, lin.cols, cnt, lin.gs, s, qa,
                w.qmm.as<uint8_t>());
  };
  for (int e = 0; e < E; ++e) {
    const int o = off[e], cnt = off[e + 1] - off[e];
    if (cnt == 0) continue;
    const DLinear *ex = &L.experts[(size_t)e * 3];
    run(ex[0], w.mq.as<int8_t>(), w.msc.as<float>(), w.msu.as<float>(), G, o, cnt, gate + (size_t)o * F);
    run(ex[1], w.mq.as<int8_t>(), w.msc.as<float>(), w.msu.as<float>(), G, o, cnt, up + (size_t)o * F);
  }
  const int total = off[E];
  if (total > 0)
    launch_silu_quant(gate, up, total, F, F, gs, w.mq.as<int8_t>(), nullptr, w.msc.as<float>(), w.msu.as<float>(),
                      s, nullptr);
  for (int e = 0; e < E; ++e) {
    const int o = off[e], cnt = off[e + 1] - off[e];
    if (cnt == 0) continue;
    run(L.experts[(size_t)e * 3 + 2], w.mq.as<int8_t>(), w.msc.as<float>(), w.msu.as<float>(), GF, o, cnt,
        w.eo.as<float>() + (size_t)o * H);
  }
  launch_moe_combine(w.hid.as<float>(), w.eo.as<float>(), w.wts.as<float>(), w.ment_of.as<int>(), m, K, H, s);
}

static void moe_block(const rai_model &md, const DLayer &L, Workspace &w, int m, hipStream_t s) {
  const rai_model_config &c = md.cfg;
  const int H = c.hidden_size, F = c.intermediate_size, E = c.num_experts, K = c.experts_per_token;
  launch_router(w.normed.as<float>(), L.router, m, H, E, K, c.norm_topk_prob, w.sel.as<int>(),
                w.wts.as<float>(), w.mlogit.as<float>(), s);
  std::vector<int> sel((size_t)m * K);
  HIP_CHECK(hipMemcpyAsync(sel.data(), w.sel.p, sel.size() * sizeof(int), hipMemcpyDeviceToHost, s));
  HIP_CHECK(hipStreamSynchronize(s));
  std::vector<std::vector<int>> tok(E), slot(E);
  for (int t = 0; t < m; ++t)
    for (int k = 0; k < K; ++k)
      if (sel[(size_t)t * K + k] >= 0) {
        tok[sel[(size_t)t * K + k]].push_back(t);
        slot[sel[(size_t)t * K + k]].push_back(k);
      }
  float *eo = w.eo.as<float>();
  for (int e = 0; e < E; ++e) {
    const int me = (int)tok[e].size();
    if (me == 0) continue;
    for (int i = 0; i < me; ++i)
      HIP_CHECK(hipMemcpyAsync(w.xg.as<float>() + (size_t)i * H, w.normed.as<float>() + (size_t)tok[e][i] * H,
                               sizeof(float) * H, hipMemcpyDeviceToDevice, s));
    const DLinear *ex = &L.experts[(size_t)e * 3];
    quantize(md, w.xg.as<float>(), me, H, w, s);
    linear(ex[0], w.xg.as<float>(), w, w.gg.as<float>(), me, s);
    linear(ex[1], w.xg.as<float>(), w, w.ug.as<float>(), me, s);
    launch_silu_mul(w.gg.as<float>(), w.ug.as<float>(), me, F, s);
    quantize(md, w.gg.as<float>(), me, F, w, s);
    linear(ex[2], w.gg.as<float>(), w, w.yg.as<float>(), me, s);
    for (int i = 0; i < me; ++i)
      HIP_CHECK(hipMemcpyAsync(eo + ((size_t)tok[e][i] * K + slot[e][i]) * H, w.yg.as<float>() + (size_t)i * H,
                               sizeof(float) * H, hipMemcpyDeviceToDevice, s));
  }
  // output.fill(0) then out += weight * value in selection order.
  launch_fill(w.mo.as<float>(), 0.0f, (size_t)m * H, s);
  std::vector<float> wt((size_t)m * K);
  HIP_CHECK(hipMemcpyAsync(wt.data(), w.wts.p, wt.size() * sizeof(float), hipMemcpyDeviceToHost, s));
  HIP_CHECK(hipStreamSynchronize(s));
  for (int k = 0; k < K; ++k) {
    // Gather slot k of every token into contiguous rows, then accumulate.
    std::vector<float> col(m);
    for (int t = 0; t < m; ++t) col[t] = sel[(size_t)t * K + k] >= 0 ? wt[(size_t)t * K + k] : 0.0f;
    HIP_CHECK(hipMemcpyAsync(w.wcol.p, col.data(), sizeof(float) * m, hipMemcpyHostToDevice, s));
    for (int t = 0; t < m; ++t)
      HIP_CHECK(hipMemcpyAsync(w.yg.as<float>() + (size_t)t * H, eo + ((size_t)t * K + k) * H, sizeof(float) * H,
                               hipMemcpyDeviceToDevice, s));
    bool any = false;
    for (int t = 0; t < m; ++t) any |= sel[(size_t)t * K + k] >= 0;
    if (any) launch_moe_accumulate(w.mo.as<float>(), w.yg.as<float>(), w.wcol.as<float>(), m, H, s);
    HIP_CHECK(hipStreamSynchronize(s));  // `col` is reused next iteration
  }
}

// Host-side checks of forward_batch (model.rs:709-725, kv_cache.rs:143-172).
static void forward_check(const rai_model &md, const rai_kv &kv, const Workspace &w, int m, size_t pos0) {
  const rai_model_config &c = md.cfg;
  if (m <= 0 || m > w.maxm) fail(RAI_E_SHAPE, "batch size exceeds the workspace");
  if (pos0 + m > c.max_context || pos0 + m > kv.cap) fail(RAI_E_RANGE, "batch position exceeds model context");
  for (int l = 0; l < kv.layers; ++l)
    if (pos0 > kv.filled[l])
      fail(RAI_E_WATERMARK, "KV store at position " + std::to_string(pos0) + " would leave a gap (filled " +
                                std::to_string(kv.filled[l]) + ")");
}

static void forward_commit(rai_kv &kv, int m, size_t pos0) {
  for (int l = 0; l < kv.layers; ++l) kv.filled[l] = std::max(kv.filled[l], pos0 + m);
}

// The launches of forward_batch (model.rs:692-963) for m tokens at positions
// pos0.. whose hidden states are in w.hid.  With a device step record `st`
// the position-dependent kernels read pos0 from it (graph replay), and the
// attention launches are sized for `span` positions (attn_span).
static void forward_enqueue(rai_model &md, rai_kv &kv, Workspace &w, int m, size_t pos0, hipStream_t s,
                            const int *st, int span = 0) {
  const rai_model_config &c = md.cfg;
  const int H = c.hidden_size, F = c.intermediate_size, hd = c.head_dim;
  const int nh = c.num_heads, nkv = c.num_kv_heads, qd = nh * hd;
  float *hid = w.hid.as<float>(), *normed = w.normed.as<float>();
  float *scores = w.attn_scores(c, kv.cap);
  const int gs = c.group_size;
  // enter_block (model.rs:319-337): RMSNorm, then one quantization of the
  // normalised rows shared by the projections that read them (the
  // reference re-quantizes per projection; the result is identical).
  auto norm_then_quant = [&](const float *wn) {
    if (fused_quant_ok(H, gs)) {
      launch_norm_quant(hid, wn, normed, m, H, c.norm_eps, gs, w.q_split.as<int8_t>(), nullptr,
                        w.qscale.as<float>(), w.qsum.as<float>(), s, mfma_acts(md, m, H, w));
    } else {
      launch_rmsnorm(hid, wn, normed, nullptr, m, H, c.norm_eps, s);
      quantize(md, normed, m, H, w, s);
    }
  };
  // One token: the projections behind a norm normalise and quantize the
  // row inside the GEMV launch (a sparse layer's MLP norm stays a launch of
  // its own: the router reads the normalised row).
  const bool norm1 = m == 1;
  for (int li = 0; li < (int)c.num_layers; ++li) {
    const DLayer &L = md.layers[li];
    const bool qkv1 = norm1 && L.qkv.rows && w4a8_norm1_path(L.qkv.rows, L.qkv.cols, L.qkv.gs);
    if (!qkv1) norm_then_quant(L.in_norm);
    float *qp, *kp, *vp;
    int q_ld, kv_ld;
    // One token: the qkv launch also rotates q and k and stores k and v
    // into the cache (rope_store in its epilogue).
    const DecRope rope{md.rope_cos, md.rope_sin, (int)pos0, st, kv.kc(li), kv.vc(li), (int)kv.cap,
                       (int)kv.vstride, nh, nkv, hd};
    const bool roped = qkv1 && kv.vstride > 0 &&
                       launch_w4a8_qkv_rope1(w.qkvb.as<float>(), L.qkv.nib, L.qkv.params, hid, L.in_norm,
                                             c.norm_eps, L.qkv.rows, L.qkv.cols, L.qkv.gs, rope, s);
    if (qkv1) {
      if (!roped)
        launch_w4a8_norm1(w.qkvb.as<float>(), nullptr, L.qkv.nib, L.qkv.params, hid, L.in_norm, c.norm_eps,
                          L.qkv.rows, L.qkv.cols, L.qkv.gs, s);
      qp = w.qkvb.as<float>();
      kp = qp + qd;
      vp = kp + nkv * hd;
      q_ld = kv_ld = L.qkv.rows;
    } else if (L.qkv.rows) {
      linear(L.qkv, normed, w, w.qkvb.as<float>(), m, s);
      qp = w.qkvb.as<float>();
      kp = qp + qd;
      vp = kp + nkv * hd;
      q_ld = kv_ld = L.qkv.rows;
    } else {
      linear(L.lin[0], normed, w, w.qb.as<float>(), m, s);
      linear(L.lin[1], normed, w, w.kb.as<float>(), m, s);
      linear(L.lin[2], normed, w, w.vb.as<float>(), m, s);
      qp = w.qb.as<float>();
      kp = w.kb.as<float>();
      vp = w.vb.as<float>();
      q_ld = qd;
      kv_ld = nkv * hd;
    }
    if (!roped)
      launch_rope_store(qp, kp, vp, md.rope_cos, md.rope_sin, (int)pos0, m, nh, nkv, hd, kv.kc(li), kv.vc(li),
                        (int)kv.cap, (int)kv.vstride, q_ld, kv_ld, s, st);
    launch_attention(qp, q_ld, kv.kc(li), kv.vc(li), (int)kv.cap, (int)kv.vstride, (int)pos0, m, nh, nkv, hd,
                     md.attn_scale, w.att.as<float>(), scores, s, st, w.err.as<int>() + 1, 7, span);
    // o_proj with the first residual add (model.rs:858-863) in its epilogue;
    // one token: the GEMV launch quantizes the attention output itself.
    const DLinear &O = L.lin[3];
    if (!(norm1 && launch_w4a8_dec(hid, hid, O.nib, O.params, nullptr, nullptr, nullptr, O.rows, O.cols, O.gs,
                                   w.att.as<float>(), nullptr, 0.0f, s))) {
      quantize(md, w.att.as<float>(), m, qd, w, s);
      linear(O, w.att.as<float>(), w, hid, m, s, hid);
    }
    const bool gu1 = norm1 && L.gate_up.rows && fused_quant_ok(F, gs) &&
                     w4a8_norm1_path(L.gate_up.rows, L.gate_up.cols, L.gate_up.gs);
    if (!gu1) norm_then_quant(L.post_norm);
    if (c.num_experts > 0 && moe_on_device(md) && m > kMfmaMaxTokens && !st) {
      moe_block_device_large(md, li, w, m, s);
    } else if (c.num_experts > 0 && moe_on_device(md)) {
      moe_block_device(md, li, w, m, s);
    } else if (c.num_experts > 0) {
      moe_block(md, L, w, m, s);
      launch_vec_add(hid, hid, w.mo.as<float>(), (size_t)m * H, s);
    } else if (gu1 && w4a8_dec_path(L.lin[6].rows, L.lin[6].cols, L.lin[6].gs) &&
               launch_w4a8_glu1(L.gate_up.nib, L.gate_up.params, hid, L.post_norm, c.norm_eps, L.gate_up.rows,
                                L.gate_up.cols, L.gate_up.gs, w.q_split.as<int8_t>(), w.qscale.as<float>(),
                                w.qsum.as<float>(), s)) {
      // One token: the gate|up launch applied the norm, SiLU-mul and the
      // quantization; down with the second residual add.
      linear(L.lin[6], w.gub.as<float>(), w, hid, m, s, hid);
    } else {
      float *gp, *up;
      int gu_ld;
      if (gu1) {
        launch_w4a8_norm1(w.gub.as<float>(), nullptr, L.gate_up.nib, L.gate_up.params, hid, L.post_norm,
                          c.norm_eps, L.gate_up.rows, L.gate_up.cols, L.gate_up.gs, s);
        gp = w.gub.as<float>();
        up = gp + F;
        gu_ld = 2 * F;
      } else if (L.gate_up.rows && fused_quant_ok(F, gs)) {
        linear(L.gate_up, normed, w, w.gub.as<float>(), m, s);
        gp = w.gub.as<float>();
        up = gp + F;
        gu_ld = 2 * F;
      } else {
        linear(L.lin[4], normed, w, w.gb.as<float>(), m, s);
        linear(L.lin[5], normed, w, w.ub.as<float>(), m, s);
        gp = w.gb.as<float>();
        up = w.ub.as<float>();
        gu_ld = F;
      }
      if (fused_quant_ok(F, gs)) {
        launch_silu_quant(gp, up, m, F, gu_ld, gs, w.q_split.as<int8_t>(), nullptr, w.qscale.as<float>(),
                          w.qsum.as<float>(), s, mfma_acts(md, m, F, w));
      } else {
        launch_silu_mul(gp, up, m, F, s);
        quantize(md, gp, m, F, w, s);
      }
      // down with the second residual add (model.rs:955-960) in its epilogue.
      linear(L.lin[6], gp, w, hid, m, s, hid);
    }
  }
}

// forward_batch: checks, launches, KV watermark.
static void forward(rai_model &md, rai_kv &kv, Workspace &w, int m, size_t pos0, hipStream_t s) {
  forward_check(md, kv, w, m, pos0);
  forward_enqueue(md, kv, w, m, pos0, s, nullptr);
  forward_commit(kv, m, pos0);
}

// hidden_to_logits_batch (model.rs:966-1033) for the m rows of w.hid.
static void logits(rai_model &md, Workspace &w, int m, hipStream_t s) {
  const rai_model_config &c = md.cfg;
  const int H = c.hidden_size, V = c.vocab_size;
  if (m > w.logit_rows) fail(RAI_E_SHAPE, "logit rows exceed the workspace");
  if (!md.tied && m == 1 &&
      w4a8_norm1_path(md.lm_head.rows, md.lm_head.cols, md.lm_head.gs)) {
    launch_w4a8_norm1(w.logits.as<float>(), nullptr, md.lm_head.nib, md.lm_head.params, w.hid.as<float>(),
                      md.final_norm, c.norm_eps, md.lm_head.rows, md.lm_head.cols, md.lm_head.gs, s);
  } else if (!md.tied) {
    if (fused_quant_ok(H, c.group_size)) {
      launch_norm_quant(w.hid.as<float>(), md.final_norm, w.normed.as<float>(), m, H, c.norm_eps, c.group_size,
                        w.q_split.as<int8_t>(), nullptr, w.qscale.as<float>(), w.qsum.as<float>(), s,
                        mfma_acts(md, m, H, w));
    } else {
      launch_rmsnorm(w.hid.as<float>(), md.final_norm, w.normed.as<float>(), nullptr, m, H, c.norm_eps, s);
      quantize(md, w.normed.as<float>(), m, H, w, s);
    }
    linear(md.lm_head, w.normed.as<float>(), w, w.logits.as<float>(), m, s);
  } else {
    launch_rmsnorm(w.hid.as<float>(), md.final_norm, w.normed.as<float>(), nullptr, m, H, c.norm_eps, s);
    launch_tied_lm_head(w.logits.as<float>(), w.normed.as<float>(), md.emb_codes, md.emb_params, V, H,
                        c.embed_group_size, m, w.hq.as<int8_t>(), w.qscale.as<float>(), w.qsum.as<float>(), s);
  }
}

static void check_tokens(const rai_model &md, const uint32_t *t, size_t n) {
  for (size_t i = 0; i < n; ++i)
    if (t[i] >= md.cfg.vocab_size) fail(RAI_E_RANGE, "token id is out of model vocabulary");
}

static void embed_tokens(rai_model &md, Workspace &w, const uint32_t *dev_tokens, int m, hipStream_t s) {
  const rai_model_config &c = md.cfg;
  launch_embed(dev_tokens, nullptr, 0, 0, m, md.emb_codes, md.emb_params, c.vocab_size, c.hidden_size,
               c.embed_group_size, c.embed_scale, w.hid.as<float>(), w.err.as<int>(), s);
}

// The workspace error words the kernels set: [0] a token id outside the
// vocabulary (embedding), [1] an attention tile hand-off wait that gave up.
// `e` holds both words as read back after the stream finished; a set word
// is cleared on the device and raised as the call's error.
static void raise_kernel_errors(Workspace &w, hipStream_t s, const int *e) {
  if (!e[0] && !e[1]) return;
  HIP_CHECK(hipMemsetAsync(w.err.p, 0, 2 * sizeof(int), s));
  HIP_CHECK(hipStreamSynchronize(s));
  if (e[1]) fail(RAI_E_HIP, "attention tile hand-off wait gave up (results discarded)");
  fail(RAI_E_RANGE, "token id is out of model vocabulary");
}

static void check_kernel_error(Workspace &w, hipStream_t s) {
  int e[2] = {0, 0};
  HIP_CHECK(hipGetLastError());
  HIP_CHECK(hipMemcpyAsync(e, w.err.p, sizeof(e), hipMemcpyDeviceToHost, s));
  HIP_CHECK(hipStreamSynchronize(s));
  raise_kernel_errors(w, s, e);
}

Workspace &model_ws(rai_model &m) {
  if (!m.ws) {
    m.ws = std::make_unique<Workspace>();
    m.ws->init(m, kChunk, 64);
  }
  return *m.ws;
}

}  // namespace rai

// -------------------------------------------------------- lookup decoder --

struct rai_lookup {
  rai_model *model = nullptr;
  rai_kv kv;
  size_t max_ctx = 0;
  rai::Workspace ws;
  DevBuf ctx;             // device context [max_ctx + 64]
  std::vector<uint32_t> ctx_host;  // mirror of ctx[0..ctx_len)
  size_t ctx_len = 0;
  DevBuf res;             // int[8]: ngram result + accept result
  // The n-gram result for the next step, searched at the end of the last
  // one (pin[0..2]): valid for that step's position, context length and
  // search parameters while the caller's context still matches.
  bool pf_valid = false;
  size_t pf_pos = 0, pf_len = 0;
  size_t pf_min = 0, pf_max = 0, pf_draft = 0;
  int *pin = nullptr;     // pinned host mirror of res + tokens (+ the step record at pin[512])
  hipStream_t stream = nullptr;
  // Step graphs: one per verify batch size m (embed, forward, logits,
  // argmax, accept) and attention span (attn_span), replayed with the
  // position in the device step record.
  DevBuf step;            // int[5] {pos0, len, start, nd, temperature bits}
  bool graphs = false;
  // Indexed by verify size m, plus (kAttnTokens + 1) times the mode (0
  // greedy, 1 exact-sampling lookup, 2 the plain sampler), plus
  // 3 (kAttnTokens + 1) per attention span index.
  std::vector<hipGraphExec_t> graph;
  std::vector<int> graph_uses;
  // Exact sampling: the decoder's StdRng (device), per-row probabilities
  // [64][V] and one row of scratch.
  DevBuf rng, probs, pscratch;
  DevBuf flags;  // [V] words for the plain sampler, zero between calls
  ~rai_lookup() {
    for (hipGraphExec_t g : graph)
      if (g) (void)hipGraphExecDestroy(g);
    if (pin) (void)hipHostFree(pin);
    if (stream) (void)hipStreamDestroy(stream);
  }
};

namespace rai {

static void kv_init(rai_kv &kv, rai_model &m, size_t max_ctx) {
  const rai_model_config &c = m.cfg;
  if (max_ctx == 0) fail(RAI_E_ARG, "KV cache context must be non-zero");
  kv.model = &m;
  kv.layers = c.num_layers;
  kv.nkv = c.num_kv_heads;
  kv.hd = c.head_dim;
  kv.cap = std::min<size_t>(max_ctx, c.max_context);
  kv.vstride = (kv.cap + 63) & ~size_t(63);
  kv.k.alloc(kv.k_bytes());
  kv.v.alloc(kv.v_bytes());
  HIP_CHECK(hipMemset(kv.k.p, 0, kv.k_bytes()));
  HIP_CHECK(hipMemset(kv.v.p, 0, kv.v_bytes()));
  kv.filled.assign(kv.layers, 0);
}

// Bring the device context in line with the caller's host context: only the
// suffix that differs from the device copy is uploaded.  Returns whether
// nothing was uploaded.
static bool sync_context(rai_lookup &d, const uint32_t *ctx, size_t len) {
  if (len > d.max_ctx) fail(RAI_E_RANGE, "context exceeds the prompt-lookup window");
  size_t same = 0;
  const size_t lim = std::min(len, d.ctx_len);
  while (same < lim && d.ctx_host[same] == ctx[same]) ++same;
  if (same < len) {
    check_tokens(*d.model, ctx + same, len - same);
    HIP_CHECK(hipMemcpyAsync(d.ctx.as<uint32_t>() + same, ctx + same, (len - same) * sizeof(uint32_t),
                             hipMemcpyHostToDevice, d.stream));
    std::copy(ctx + same, ctx + len, d.ctx_host.begin() + same);
  }
  d.ctx_len = len;
  return same == len;
}

// One decode step: LookupDecoder::step (lookup.rs:260-425).  With
// search = false the n-gram search is skipped and the step is decode_one
// (lookup.rs:428-455): the plain decode loop of `rai run` (run.rs:692-735),
// on the same one-token step graph; `plain` (then) selects the token with
// the repetition penalty and sample_token's whole SamplerConfig
// (sampler.rs:47-199) instead of argmax.
static void lookup_step(rai_lookup &d, size_t pos, const uint32_t *context, size_t len,
                        const rai_lookup_config &cfg, uint32_t *out, size_t cap, rai_lookup_metrics &met,
                        bool search = true, const rai_sampler_config *plain = nullptr) {
  rai_model &md = *d.model;
  const rai_model_config &c = md.cfg;
  // validate_lookup_config (lookup.rs:457-475), greedy variant.
  if (cfg.max_draft == 0) fail(RAI_E_ARG, "prompt-lookup max_draft must be non-zero");
  if (cfg.min_ngram < 1 || cfg.min_ngram > cfg.max_ngram)
    fail(RAI_E_ARG, "prompt-lookup requires 1 <= min_ngram <= max_ngram");
  // Above 1e-6 the step samples exactly (lookup.rs:359-403) from the
  // decoder's generator; at or below it, greedy acceptance.
  if (!std::isfinite(cfg.temperature)) fail(RAI_E_ARG, "temperature must be finite");
  const bool sampled = cfg.temperature > 1e-6f;
  // The device context keeps 64 slots past max_ctx for the accepted tokens
  // and the workspace holds 64 logit rows: the verify batch is at most 64.
  if (cfg.max_draft > 63) fail(RAI_E_ARG, "max_draft above 63 is not supported");
  if (len == 0) fail(RAI_E_ARG, "prompt-lookup step requires a non-empty context");
  if (pos >= d.max_ctx) fail(RAI_E_RANGE, "decode position exceeds the context window");
  if (cap < cfg.max_draft + 1) fail(RAI_E_SHAPE, "output buffer must hold max_draft + 1 tokens");
  if (len > d.max_ctx) fail(RAI_E_RANGE, "context exceeds the prompt-lookup window");
  const bool unchanged = sync_context(d, context, len);
  // The previous step searched this step's draft already (pin[0..2]) when
  // the context, position and search parameters are the ones it assumed.
  const bool prefetched = d.pf_valid && unchanged && len == d.pf_len && pos == d.pf_pos &&
                          cfg.min_ngram == d.pf_min && cfg.max_ngram == d.pf_max && cfg.max_draft == d.pf_draft;
  d.pf_valid = false;
  hipStream_t s = d.stream;
  const size_t budget = d.max_ctx > pos + 1 ? d.max_ctx - pos - 1 : 0;
  int *res = d.res.as<int>();
  int nd = 0, start = 0, ngram = 0;
  if (budget > 0 && search) {
    if (!prefetched) {
      launch_ngram(d.ctx.as<uint32_t>(), (int)len, (int)cfg.min_ngram, (int)cfg.max_ngram,
                   (int)std::min(cfg.max_draft, budget), res, s);
      HIP_CHECK(hipMemcpyAsync(d.pin, res, 3 * sizeof(int), hipMemcpyDeviceToHost, s));
      HIP_CHECK(hipStreamSynchronize(s));
    }
    ngram = d.pin[0];
    start = d.pin[1];
    nd = ngram ? d.pin[2] : 0;
  }
  const int m = nd + 1;  // verify [last, draft...] or the single decode_one token
  forward_check(md, d.kv, d.ws, m, pos);
  // The attention span a graph of this step is captured for: every position
  // up to it replays the same graph.
  const int span = attn_span((int)d.kv.cap, (int)pos + m);
  auto enqueue = [&](const int *st) {
    launch_embed(nullptr, d.ctx.as<uint32_t>(), (int)len - 1, start, m, md.emb_codes, md.emb_params,
                 c.vocab_size, c.hidden_size, c.embed_group_size, c.embed_scale, d.ws.hid.as<float>(),
                 d.ws.err.as<int>(), s, st);
    forward_enqueue(md, d.kv, d.ws, m, pos, s, st, span);
    logits(md, d.ws, m, s);
    if (plain) {
      launch_sample_plain(d.ws.logits.as<float>(), c.vocab_size, d.ctx.as<uint32_t>(), (int)len,
                          plain->temperature, (int)std::min<size_t>(plain->top_k, INT32_MAX), plain->top_p,
                          plain->repetition_penalty, d.rng.as<RngState>(), d.pscratch.as<float>(),
                          d.flags.as<uint32_t>(), nullptr, res + 4, s, st);
    } else if (sampled) {
      launch_sample(d.ws.logits.as<float>(), d.probs.as<float>(), c.vocab_size, d.ctx.as<uint32_t>(), (int)len,
                    start, nd, cfg.temperature, d.rng.as<RngState>(), d.pscratch.as<float>(), res + 4, s, st, m);
    } else {
      launch_argmax(d.ws.logits.as<float>(), m, c.vocab_size, d.ws.am.as<uint32_t>(), s);
      launch_accept(d.ws.am.as<uint32_t>(), d.ctx.as<uint32_t>(), (int)len, start, nd, res + 4, s, st);
    }
    // The next step's n-gram search over the extended context, so that a
    // caller continuing from this step's tokens needs one host round trip
    // per step.
    launch_ngram_next(d.ctx.as<uint32_t>(), (int)len, (int)pos, (int)cfg.min_ngram, (int)cfg.max_ngram,
                      (int)cfg.max_draft, (int)d.max_ctx, res + 4, res, s, st);
  };
  HIP_CHECK(hipGetLastError());  // nothing pending from earlier launches
  if (d.graphs && m <= kAttnTokens) {
    int *sh = d.pin + 512;
    sh[0] = (int)pos;
    sh[1] = (int)len;
    sh[2] = start;
    sh[3] = nd;
    std::memcpy(&sh[4], &cfg.temperature, sizeof(float));
    sh[5] = (int)cfg.min_ngram;
    sh[6] = (int)cfg.max_ngram;
    sh[7] = (int)cfg.max_draft;
    sh[8] = plain ? (int)std::min<size_t>(plain->top_k, INT32_MAX) : 0;
    std::memcpy(&sh[9], plain ? &plain->top_p : &cfg.temperature, sizeof(float));
    std::memcpy(&sh[10], plain ? &plain->repetition_penalty : &cfg.temperature, sizeof(float));
    if (plain) std::memcpy(&sh[4], &plain->temperature, sizeof(float));
    HIP_CHECK(hipMemcpyAsync(d.step.p, sh, 11 * sizeof(int), hipMemcpyHostToDevice, s));
    const int *st = d.step.as<int>();
    const int mode = plain ? 2 : sampled ? 1 : 0;
    const int gi = m + (kAttnTokens + 1) * mode + 3 * (kAttnTokens + 1) * attn_span_index((int)pos + m);
    if (d.graph[gi]) {
      HIP_CHECK(hipGraphLaunch(d.graph[gi], s));
    } else if (d.graph_uses[gi]++ == 0) {
      enqueue(st);  // first use: eager (sets kernel attributes, sizes scratch)
      HIP_CHECK(hipGetLastError());
    } else {
      hipGraph_t g = nullptr;
      HIP_CHECK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
      enqueue(st);
      const hipError_t le = hipGetLastError();
      const hipError_t ce = hipStreamEndCapture(s, &g);
      if (le != hipSuccess || ce != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        HIP_CHECK(le);
        HIP_CHECK(ce);
      }
      hipGraphExec_t ge = nullptr;
      const hipError_t ie = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
      (void)hipGraphDestroy(g);
      HIP_CHECK(ie);
      d.graph[gi] = ge;
      HIP_CHECK(hipGraphLaunch(ge, s));
    }
  } else {
    enqueue(nullptr);
    HIP_CHECK(hipGetLastError());
  }
  HIP_CHECK(hipMemcpyAsync(d.pin, res, 3 * sizeof(int), hipMemcpyDeviceToHost, s));
  HIP_CHECK(hipMemcpyAsync(d.pin + 4, res + 4, 2 * sizeof(int), hipMemcpyDeviceToHost, s));
  HIP_CHECK(hipMemcpyAsync(d.pin + 6, d.ws.err.p, 2 * sizeof(int), hipMemcpyDeviceToHost, s));
  HIP_CHECK(hipMemcpyAsync(d.pin + 8, d.ctx.as<uint32_t>() + len, (size_t)m * sizeof(uint32_t),
                           hipMemcpyDeviceToHost, s));
  HIP_CHECK(hipStreamSynchronize(s));
  if (d.pin[6] || d.pin[7]) {
    // The step's outputs are not trusted: the KV rows it wrote stay above
    // the watermark and the device context past len is ignored.
    d.ctx_len = std::min(d.ctx_len, len);
    const int e[2] = {d.pin[6], d.pin[7]};
    raise_kernel_errors(d.ws, s, e);
  }
  forward_commit(d.kv, m, pos);
  const int acc = d.pin[4], prod = d.pin[5];
  for (int i = 0; i < prod; ++i) out[i] = (uint32_t)d.pin[8 + i];
  // The accept kernel already appended the produced tokens to the device
  // context; mirror that so the caller's extended context needs no upload.
  for (int i = 0; i < prod; ++i) d.ctx_host[len + i] = out[i];
  d.ctx_len = len + prod;
  // kv_cache.truncate(pos + produced) (lookup.rs:411).
  for (auto &f : d.kv.filled) f = std::min(f, pos + (size_t)prod);
  d.pf_valid = true;
  d.pf_pos = pos + (size_t)prod;
  d.pf_len = len + (size_t)prod;
  d.pf_min = cfg.min_ngram;
  d.pf_max = cfg.max_ngram;
  d.pf_draft = cfg.max_draft;
  met.accepted = nd ? acc : 0;
  met.drafted = nd;
  met.produced = prod;
  met.matched_ngram = ngram;
  met.accept_rate = nd ? (float)acc / (float)nd : 0.0f;
}

static void lookup_prefill(rai_lookup &d, const uint32_t *prompt, size_t n, size_t &pos_out) {
  rai_model &md = *d.model;
  if (n == 0) fail(RAI_E_ARG, "prompt must contain at least one token");
  if (n > d.max_ctx) fail(RAI_E_RANGE, "prompt exceeds the prompt-lookup context window");
  check_tokens(md, prompt, n);
  d.pf_valid = false;
  sync_context(d, prompt, n);
  const size_t cnt = n - 1;
  for (size_t p = 0; p < cnt; p += kChunk) {
    const int m = (int)std::min<size_t>(kChunk, cnt - p);
    launch_embed(d.ctx.as<uint32_t>() + p, nullptr, 0, 0, m, md.emb_codes, md.emb_params, md.cfg.vocab_size,
                 md.cfg.hidden_size, md.cfg.embed_group_size, md.cfg.embed_scale, d.ws.hid.as<float>(),
                 d.ws.err.as<int>(), d.stream);
    forward(md, d.kv, d.ws, m, p, d.stream);
  }
  try {
    check_kernel_error(d.ws, d.stream);
  } catch (...) {
    for (auto &f : d.kv.filled) f = 0;  // nothing of this prefill is trusted
    throw;
  }
  pos_out = cnt;
}

}  // namespace rai

// ================================================================ C ABI ==

extern "C" {

const char *rai_last_error(void) { return rai::g_last_error.c_str(); }

int rai_device_info(char *name, size_t name_len, int *cus) {
  RAI_API_BODY({
    hipDeviceProp_t p;
    int dev = 0;
    HIP_CHECK(hipGetDevice(&dev));
    HIP_CHECK(hipGetDeviceProperties(&p, dev));
    if (name && name_len) {
      std::snprintf(name, name_len, "%s (%s)", p.name, p.gcnArchName);
    }
    if (cus) *cus = p.multiProcessorCount;
  });
}

int rai_model_from_buffer(const void *data, size_t len, int max_groups, rai_model **out) {
  RAI_API_BODY({
    if (!data || !out) rai::fail(RAI_E_ARG, "null argument");
    auto m = std::make_unique<rai_model>();
    rai::upload_model(*m, (const uint8_t *)data, len, max_groups);
    *out = m.release();
  });
}

int rai_model_open(const char *path, int max_groups, rai_model **out) {
  RAI_API_BODY({
    if (!path || !out) rai::fail(RAI_E_ARG, "null argument");
    std::ifstream f(path, std::ios::binary | std::ios::ate);
    if (!f) rai::fail(RAI_E_IO, std::string("opening ") + path);
    const std::streamsize n = f.tellg();
    if (n < 0) rai::fail(RAI_E_IO, std::string("stat ") + path);
    if ((uint64_t)n > (64ull << 30)) rai::fail(RAI_E_FORMAT, "model file is too large");
    std::vector<uint8_t> buf((size_t)n);
    f.seekg(0);
    if (!f.read((char *)buf.data(), n)) rai::fail(RAI_E_IO, std::string("reading ") + path);
    auto m = std::make_unique<rai_model>();
    rai::upload_model(*m, buf.data(), buf.size(), max_groups);
    *out = m.release();
  });
}

void rai_model_free(rai_model *m) { delete m; }

int rai_model_get_config(const rai_model *m, rai_model_config *out) {
  RAI_API_BODY({
    if (!m || !out) rai::fail(RAI_E_ARG, "null argument");
    *out = m->cfg;
  });
}

int rai_model_weight_bytes(const rai_model *m, uint64_t *out) {
  RAI_API_BODY({
    if (!m || !out) rai::fail(RAI_E_ARG, "null argument");
    *out = m->weight_bytes;
  });
}

int rai_kv_create(rai_model *m, size_t max_ctx, rai_kv **out) {
  RAI_API_BODY({
    if (!m || !out) rai::fail(RAI_E_ARG, "null argument");
    auto kv = std::make_unique<rai_kv>();
    rai::kv_init(*kv, *m, max_ctx);
    *out = kv.release();
  });
}

void rai_kv_free(rai_kv *kv) { delete kv; }

int rai_kv_truncate(rai_kv *kv, size_t len) {
  RAI_API_BODY({
    if (!kv) rai::fail(RAI_E_ARG, "null argument");
    for (auto &f : kv->filled) f = std::min(f, len);
  });
}

int rai_kv_filled(const rai_kv *kv, size_t layer, size_t *out) {
  RAI_API_BODY({
    if (!kv || !out) rai::fail(RAI_E_ARG, "null argument");
    if (layer >= kv->filled.size()) rai::fail(RAI_E_ARG, "layer index out of range");
    *out = kv->filled[layer];
  });
}

int rai_kv_clear(rai_kv *kv) {
  RAI_API_BODY({
    if (!kv) rai::fail(RAI_E_ARG, "null argument");
    HIP_CHECK(hipMemset(kv->k.p, 0, kv->k_bytes()));
    HIP_CHECK(hipMemset(kv->v.p, 0, kv->v_bytes()));
    std::fill(kv->filled.begin(), kv->filled.end(), 0);
  });
}

int rai_kv_read(const rai_kv *kv, size_t layer, size_t head, size_t pos, int which, float *out) {
  RAI_API_BODY({
    if (!kv || !out) rai::fail(RAI_E_ARG, "null argument");
    if (layer >= (size_t)kv->layers || head >= (size_t)kv->nkv) rai::fail(RAI_E_ARG, "KV cache head is out of range");
    if (pos >= kv->filled[layer])
      rai::fail(RAI_E_WATERMARK, "KV read at unwritten position " + std::to_string(pos) + " (filled " +
                                     std::to_string(kv->filled[layer]) + ")");
    // The cache is written on the decoders' own (non-blocking) streams:
    // wait for all of their work before copying.
    HIP_CHECK(hipDeviceSynchronize());
    if (which == 0) {
      const float *base = kv->kc((int)layer);
      HIP_CHECK(hipMemcpy(out, base + (head * kv->cap + pos) * kv->hd, kv->hd * sizeof(float), hipMemcpyDeviceToHost));
    } else {
      // d-major V: the row's hd values are vstride floats apart.
      const float *base = kv->vc((int)layer) + head * kv->hd * kv->vstride + pos;
      HIP_CHECK(hipMemcpy2D(out, sizeof(float), base, kv->vstride * sizeof(float), sizeof(float), kv->hd,
                            hipMemcpyDeviceToHost));
    }
  });
}

int rai_embed_token(rai_model *m, size_t token, float *out) {
  RAI_API_BODY({
    if (!m || !out) rai::fail(RAI_E_ARG, "null argument");
    if (token >= m->cfg.vocab_size) rai::fail(RAI_E_RANGE, "token id is out of model vocabulary");
    rai::Workspace &w = rai::model_ws(*m);
    const uint32_t t = (uint32_t)token;
    HIP_CHECK(hipMemcpyAsync(w.am.p, &t, 4, hipMemcpyHostToDevice, m->stream));
    rai::embed_tokens(*m, w, w.am.as<uint32_t>(), 1, m->stream);
    HIP_CHECK(hipMemcpyAsync(out, w.hid.p, sizeof(float) * m->cfg.hidden_size, hipMemcpyDeviceToHost, m->stream));
    rai::check_kernel_error(w, m->stream);
  });
}

int rai_forward_batch(rai_model *m, rai_kv *kv, float *hiddens, const size_t *positions, size_t batch) {
  RAI_API_BODY({
    if (!m || !kv || !hiddens || !positions) rai::fail(RAI_E_ARG, "null argument");
    if (kv->model != m) rai::fail(RAI_E_ARG, "KV cache belongs to another model");
    if (batch == 0) rai::fail(RAI_E_ARG, "batch must contain at least one token");
    for (size_t b = 0; b < batch; ++b) {
      if (positions[b] >= m->cfg.max_context) rai::fail(RAI_E_RANGE, "batch position exceeds model context");
      if (b && positions[b] != positions[b - 1] + 1)
        rai::fail(RAI_E_ARG, "batch positions must be strictly consecutive and ascending");
    }
    rai::Workspace &w = rai::model_ws(*m);
    const size_t H = m->cfg.hidden_size;
    const std::vector<size_t> filled0 = kv->filled;
    for (size_t b0 = 0; b0 < batch; b0 += rai::kChunk) {
      const int mm = (int)std::min<size_t>(rai::kChunk, batch - b0);
      HIP_CHECK(hipMemcpyAsync(w.hid.p, hiddens + b0 * H, sizeof(float) * H * mm, hipMemcpyHostToDevice, m->stream));
      rai::forward(*m, *kv, w, mm, positions[b0], m->stream);
      HIP_CHECK(hipMemcpyAsync(hiddens + b0 * H, w.hid.p, sizeof(float) * H * mm, hipMemcpyDeviceToHost, m->stream));
    }
    try {
      rai::check_kernel_error(w, m->stream);
    } catch (...) {
      kv->filled = filled0;  // the batch's KV rows are not trusted
      throw;
    }
  });
}

int rai_forward_from_hidden(rai_model *m, rai_kv *kv, float *hidden, size_t pos, int store_kv) {
  if (!store_kv) {
    rai::set_last_error("probe passes (store_kv = 0) are not part of the lookup path");
    return RAI_E_UNSUPPORTED;
  }
  return rai_forward_batch(m, kv, hidden, &pos, 1);
}

int rai_hidden_to_logits_batch(rai_model *m, const float *hiddens, float *out, size_t batch) {
  RAI_API_BODY({
    if (!m || !hiddens || !out) rai::fail(RAI_E_ARG, "null argument");
    if (batch == 0) rai::fail(RAI_E_ARG, "batch must contain at least one token");
    rai::Workspace &w = rai::model_ws(*m);
    const size_t H = m->cfg.hidden_size, V = m->cfg.vocab_size;
    for (size_t b0 = 0; b0 < batch; b0 += (size_t)w.logit_rows) {
      const int mm = (int)std::min<size_t>(w.logit_rows, batch - b0);
      HIP_CHECK(hipMemcpyAsync(w.hid.p, hiddens + b0 * H, sizeof(float) * H * mm, hipMemcpyHostToDevice, m->stream));
      rai::logits(*m, w, mm, m->stream);
      HIP_CHECK(hipMemcpyAsync(out + b0 * V, w.logits.p, sizeof(float) * V * mm, hipMemcpyDeviceToHost, m->stream));
    }
    HIP_CHECK(hipStreamSynchronize(m->stream));
  });
}

int rai_hidden_to_logits(rai_model *m, const float *hidden, float *out) {
  return rai_hidden_to_logits_batch(m, hidden, out, 1);
}

int rai_w4a8_matmul_dev(float *out, const uint8_t *nib, const uint8_t *params, const float *x, size_t rows,
                        size_t cols, size_t m, size_t gs, void *stream) {
  RAI_API_BODY({
    // validate_weight_buffers (gemm.rs:1169-1213).
    if (!out || !nib || !params || !x) rai::fail(RAI_E_ARG, "null argument");
    if (rows == 0) rai::fail(RAI_E_SHAPE, "rows must be non-zero");
    if (cols == 0 || cols % 2) rai::fail(RAI_E_SHAPE, "cols must be non-zero and even");
    if (gs == 0 || gs % 2) rai::fail(RAI_E_SHAPE, "group_size must be non-zero and even");
    if (m == 0) rai::fail(RAI_E_SHAPE, "num_tokens must be non-zero");
    if (rows > INT32_MAX || cols > INT32_MAX || m > INT32_MAX) rai::fail(RAI_E_SHAPE, "dimensions overflow");
    hipStream_t s = (hipStream_t)stream;
    const size_t groups = rai::ceil_div(cols, gs);
    rai::DevBuf qn, qs, sc, su;
    qn.alloc(m * cols);
    qs.alloc(m * cols);
    sc.alloc(m * groups * 4);
    su.alloc(m * groups * 4);
    rai::launch_quantize(x, (int)m, (int)cols, (int)gs, qn.as<int8_t>(), qs.as<int8_t>(), sc.as<float>(),
                         su.as<float>(), s);
    rai::DevBuf qa, mm;
    const bool mfma = rai::w4a8_mfma_path((int)rows, (int)cols, (int)m, (int)gs);
    if (mfma) {
      qa.alloc(sizeof(_Float16) * rai::qa_pack_halves((int)m, (int)cols));
      rai::launch_qa_pack(qs.as<int8_t>(), (int)m, (int)cols, qa.as<_Float16>(), s);
    }
    if (rai::w4a8_mm_path((int)rows, (int)cols, (int)m, (int)gs)) mm.alloc(rai::mm_pack_bytes((int)m, (int)cols));
    rai::launch_w4a8(out, nullptr, nib, params, x, qn.as<int8_t>(), qs.as<int8_t>(), sc.as<float>(),
                     su.as<float>(), (int)rows, (int)cols, (int)m, (int)gs, s, mfma ? qa.as<_Float16>() : nullptr,
                     mm.as<uint8_t>());
    HIP_CHECK(hipGetLastError());
    HIP_CHECK(hipStreamSynchronize(s));  // scratch is freed on return
  });
}

// w4a8_fused_qkv / w4a8_fused_gate_up (gemm.rs:1386-1703): the projections'
// checks (validate_projection, gemm.rs:1215-1226, and the agreement of
// cols and group_size), one quantization of the input row, then each
// projection's one-token GEMV on the shared activations.
static void fused_projections(float *const *outs, const rai_qlinear *const *lin, const char *const *names, int n,
                              const float *x, void *stream) {
  if (!x) rai::fail(RAI_E_ARG, "null argument");
  for (int i = 0; i < n; ++i) {
    if (!outs[i] || !lin[i] || !lin[i]->nibbles || !lin[i]->params) rai::fail(RAI_E_ARG, "null argument");
    const rai_qlinear &L = *lin[i];
    if (L.rows == 0) rai::fail(RAI_E_SHAPE, "rows must be non-zero");
    if (L.cols == 0 || L.cols % 2) rai::fail(RAI_E_SHAPE, "cols must be non-zero and even");
    if (L.group_size == 0 || L.group_size % 2) rai::fail(RAI_E_SHAPE, "group_size must be non-zero and even");
    if (L.rows > INT32_MAX || L.cols > INT32_MAX) rai::fail(RAI_E_SHAPE, "dimensions overflow");
  }
  for (int i = 1; i < n; ++i) {
    if (lin[i]->cols != lin[0]->cols) rai::fail(RAI_E_SHAPE, std::string(names[i]) + " column mismatch");
    if (lin[i]->group_size != lin[0]->group_size) rai::fail(RAI_E_SHAPE, std::string(names[i]) + " group mismatch");
  }
  hipStream_t s = (hipStream_t)stream;
  const size_t cols = lin[0]->cols, gs = lin[0]->group_size, groups = rai::ceil_div(cols, gs);
  rai::DevBuf qn, qs, sc, su;
  qn.alloc(cols);
  qs.alloc(cols);
  sc.alloc(groups * 4);
  su.alloc(groups * 4);
  rai::launch_quantize(x, 1, (int)cols, (int)gs, qn.as<int8_t>(), qs.as<int8_t>(), sc.as<float>(), su.as<float>(), s);
  for (int i = 0; i < n; ++i)
    rai::launch_w4a8(outs[i], nullptr, lin[i]->nibbles, lin[i]->params, x, qn.as<int8_t>(), qs.as<int8_t>(),
                     sc.as<float>(), su.as<float>(), (int)lin[i]->rows, (int)cols, 1, (int)gs, s, nullptr, nullptr);
  HIP_CHECK(hipGetLastError());
  HIP_CHECK(hipStreamSynchronize(s));  // scratch is freed on return
}

int rai_w4a8_fused_qkv_dev(float *q_out, float *k_out, float *v_out, const rai_qlinear *q, const rai_qlinear *k,
                           const rai_qlinear *v, const float *x, void *stream) {
  RAI_API_BODY({
    float *const outs[3] = {q_out, k_out, v_out};
    const rai_qlinear *const lin[3] = {q, k, v};
    const char *const names[3] = {"Q", "Q/K", "Q/V"};
    fused_projections(outs, lin, names, 3, x, stream);
  });
}

int rai_w4a8_fused_gate_up_dev(float *gate_out, float *up_out, const rai_qlinear *gate, const rai_qlinear *up,
                               const float *x, void *stream) {
  RAI_API_BODY({
    float *const outs[2] = {gate_out, up_out};
    const rai_qlinear *const lin[2] = {gate, up};
    const char *const names[2] = {"gate", "gate/up"};
    fused_projections(outs, lin, names, 2, x, stream);
  });
}

// ------------------------------------------------- allocation-free GEMM --
//
// Scratch of rai_w4a8_matmul_noalloc_dev: one static device array per GPU,
// held until the process ends.  Host code never uses the array's name as a
// device address (in host code it names a host-side stand-in); it uses the
// address hipGetSymbolAddress returns on each device, looked up once per
// device on the first call there.  Layout (bytes): q_nat [m*cols], q_split
// [m*cols], scales [m*groups] f32, sums [m*groups] f32, matrix-core
// activations (2..64 tokens), the matrix-core GEMM's activation records
// (more than 64 tokens at group 32: at most ceil(m/32) * cols/32 * 2304
// bytes, which for m > 64 and m * cols <= 2^20 stays below 3/65 * 72 * 2^20).
namespace rai {
constexpr size_t kNaTokenCols = size_t(1) << 20;  // m * cols
constexpr size_t kNaGroups = size_t(1) << 16;     // m * ceil(cols / gs)
constexpr size_t kNaQaBytes = size_t(2) << 20;
constexpr size_t kNaMmBytes = size_t(7) << 19;  // 3.5 MiB
constexpr size_t kNaScratchBytes = 2 * kNaTokenCols + 8 * kNaGroups + kNaQaBytes + kNaMmBytes;
constexpr int kNaMaxDevices = 64;
}  // namespace rai

static __device__ __align__(256) uint8_t scratch[rai::kNaScratchBytes];

namespace rai {

static std::mutex g_na_mutex;
static void *g_na_scratch[kNaMaxDevices] = {};

// The device address of `scratch` on the current device.
static uint8_t *noalloc_scratch() {
  int dev = 0;
  HIP_CHECK(hipGetDevice(&dev));
  if (dev < 0 || dev >= kNaMaxDevices) fail(RAI_E_ARG, "device index out of range");
  std::lock_guard<std::mutex> lk(g_na_mutex);
  if (!g_na_scratch[dev]) {
    void *p = nullptr;
    HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) fail(RAI_E_HIP, "hipGetSymbolAddress returned no address for the scratch array");
    g_na_scratch[dev] = p;
  }
  return static_cast<uint8_t *>(g_na_scratch[dev]);
}

}  // namespace rai

int rai_w4a8_matmul_noalloc_dev(float *out, const uint8_t *nib, const uint8_t *params, const float *x, size_t rows,
                                size_t cols, size_t m, size_t gs, void *stream) {
  RAI_API_BODY({
    if (!out || !nib || !params || !x) rai::fail(RAI_E_ARG, "null argument");
    if (rows == 0) rai::fail(RAI_E_SHAPE, "rows must be non-zero");
    if (cols == 0 || cols % 2) rai::fail(RAI_E_SHAPE, "cols must be non-zero and even");
    if (gs == 0 || gs % 2) rai::fail(RAI_E_SHAPE, "group_size must be non-zero and even");
    if (m == 0) rai::fail(RAI_E_SHAPE, "num_tokens must be non-zero");
    if (rows > INT32_MAX || cols > INT32_MAX || m > INT32_MAX) rai::fail(RAI_E_SHAPE, "dimensions overflow");
    const size_t groups = rai::ceil_div(cols, gs);
    if (m > rai::kNaTokenCols / cols || m * groups > rai::kNaGroups)
      rai::fail(RAI_E_SHAPE, "num_tokens * cols exceeds the allocation-free scratch (at most " +
                                 std::to_string(rai::kNaTokenCols) + " token columns and " +
                                 std::to_string(rai::kNaGroups) + " token groups)");
    const bool mfma = rai::w4a8_mfma_path((int)rows, (int)cols, (int)m, (int)gs);
    if (mfma && sizeof(_Float16) * rai::qa_pack_halves((int)m, (int)cols) > rai::kNaQaBytes)
      rai::fail(RAI_E_SHAPE, "activation tile exceeds the allocation-free scratch");
    const bool mm = rai::w4a8_mm_path((int)rows, (int)cols, (int)m, (int)gs);
    if (mm && rai::mm_pack_bytes((int)m, (int)cols) > rai::kNaMmBytes)
      rai::fail(RAI_E_SHAPE, "activation records exceed the allocation-free scratch");
    uint8_t *base = rai::noalloc_scratch();
    int8_t *qn = reinterpret_cast<int8_t *>(base);
    int8_t *qs = reinterpret_cast<int8_t *>(base + rai::kNaTokenCols);
    float *sc = reinterpret_cast<float *>(base + 2 * rai::kNaTokenCols);
    float *su = sc + rai::kNaGroups;
    _Float16 *qa = reinterpret_cast<_Float16 *>(base + 2 * rai::kNaTokenCols + 8 * rai::kNaGroups);
    uint8_t *mmp = base + 2 * rai::kNaTokenCols + 8 * rai::kNaGroups + rai::kNaQaBytes;
    hipStream_t s = (hipStream_t)stream;
    // Every scratch byte a kernel reads is written earlier in this call (the
    // pack writes the padding rows of the last token group as zeros), so the
    // previous call's contents never reach the output.
    rai::launch_quantize(x, (int)m, (int)cols, (int)gs, qn, qs, sc, su, s);
    if (mfma) rai::launch_qa_pack(qs, (int)m, (int)cols, qa, s);
    rai::launch_w4a8(out, nullptr, nib, params, x, qn, qs, sc, su, (int)rows, (int)cols, (int)m, (int)gs, s,
                     mfma ? qa : nullptr, mm ? mmp : nullptr);
    HIP_CHECK(hipGetLastError());
  });
}

int rai_w4a8_time_dev(float *out, const uint8_t *nib, const uint8_t *params, const float *x, size_t rows,
                      size_t cols, size_t m, size_t gs, size_t copies, int iters, float *avg_ms) {
  RAI_API_BODY({
    if (!out || !nib || !params || !x || !avg_ms) rai::fail(RAI_E_ARG, "null argument");
    if (rows == 0 || cols == 0 || cols % 2 || gs == 0 || gs % 2 || m == 0 || iters <= 0 || copies == 0)
      rai::fail(RAI_E_SHAPE, "invalid shape");
    const size_t groups = rai::ceil_div(cols, gs);
    rai::DevBuf qn, qs, sc, su;
    qn.alloc(m * cols);
    qs.alloc(m * cols);
    sc.alloc(m * groups * 4);
    su.alloc(m * groups * 4);
    hipStream_t s;
    HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    hipEvent_t e0, e1;
    HIP_CHECK(hipEventCreate(&e0));
    HIP_CHECK(hipEventCreate(&e1));
    rai::launch_quantize(x, (int)m, (int)cols, (int)gs, qn.as<int8_t>(), qs.as<int8_t>(), sc.as<float>(),
                         su.as<float>(), s);
    rai::DevBuf qa, mm;
    const bool mfma = rai::w4a8_mfma_path((int)rows, (int)cols, (int)m, (int)gs);
    if (mfma) {
      qa.alloc(sizeof(_Float16) * rai::qa_pack_halves((int)m, (int)cols));
      rai::launch_qa_pack(qs.as<int8_t>(), (int)m, (int)cols, qa.as<_Float16>(), s);
    }
    if (rai::w4a8_mm_path((int)rows, (int)cols, (int)m, (int)gs)) mm.alloc(rai::mm_pack_bytes((int)m, (int)cols));
    const size_t nib_bytes = rows * cols / 2, par_bytes = rows * groups * 4;
    // The parameters' tile-layout copies, as a loaded model holds them.
    rai::DevBuf tiled;
    if (mfma && rai::params_tile16_ok((int)rows, (int)cols, (int)gs)) {
      tiled.alloc(copies * par_bytes);
      for (size_t c = 0; c < copies; ++c)
        rai::launch_params_tile16(params + c * par_bytes, (int)rows, (int)cols, tiled.as<uint8_t>() + c * par_bytes,
                                  s);
      HIP_CHECK(hipGetLastError());
    }
    auto run = [&](size_t c) {
      rai::launch_w4a8(out, nullptr, nib + c * nib_bytes, params + c * par_bytes, x, qn.as<int8_t>(),
                       qs.as<int8_t>(), sc.as<float>(), su.as<float>(), (int)rows, (int)cols, (int)m, (int)gs, s,
                       mfma ? qa.as<_Float16>() : nullptr, mm.as<uint8_t>(),
                       tiled.p ? tiled.as<uint8_t>() + c * par_bytes : nullptr);
    };
    run(0);  // warm-up
    HIP_CHECK(hipEventRecord(e0, s));
    for (int i = 0; i < iters; ++i) run((size_t)(i + 1) % copies);
    HIP_CHECK(hipEventRecord(e1, s));
    HIP_CHECK(hipEventSynchronize(e1));
    float ms = 0.0f;
    HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
    *avg_ms = ms / iters;
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    (void)hipStreamDestroy(s);
  });
}

int rai_attention_time_dev(const float *q, const float *kc, const float *vc, size_t cap, size_t pos, size_t m,
                           size_t nh, size_t nkv, size_t hd, size_t copies, int iters, float *ms3) {
  RAI_API_BODY({
    if (!q || !kc || !vc || !ms3) rai::fail(RAI_E_ARG, "null argument");
    if (m == 0 || m > (size_t)rai::kAttnTokens || nkv == 0 || nh % nkv || hd == 0 || hd % 8 || copies == 0 ||
        iters <= 0)
      rai::fail(RAI_E_SHAPE, "invalid attention shape");
    if (pos + m > cap) rai::fail(RAI_E_RANGE, "positions exceed the cache");
    const size_t vstride = (cap + 63) & ~size_t(63);
    const size_t kbytes = nkv * cap * hd, vbytes = nkv * hd * vstride;  // floats per copy
    rai::DevBuf out, scores, err;
    out.alloc(sizeof(float) * m * nh * hd);
    scores.alloc(sizeof(float) * rai::attention_scores_floats((int)m, (int)nh, (int)(pos + m)));
    err.alloc(sizeof(int));
    hipStream_t s;
    HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    HIP_CHECK(hipMemsetAsync(err.p, 0, sizeof(int), s));
    // A full warm-up pass, then each stage on its own, `iters` launches back
    // to back between two events (stage inputs are what the previous pass
    // left in the buffers), rotating the K / V copies.
    hipEvent_t ev[2];
    for (auto &e : ev) HIP_CHECK(hipEventCreate(&e));
    const float scale = 1.0f / std::sqrt((float)hd);
    auto run = [&](size_t c, int stages) {
      rai::launch_attention(q, (int)(nh * hd), kc + c * kbytes, vc + c * vbytes, (int)cap, (int)vstride, (int)pos,
                            (int)m, (int)nh, (int)nkv, (int)hd, scale, out.as<float>(), scores.as<float>(), s,
                            nullptr, err.as<int>(), stages);
    };
    run(0, 7);
    HIP_CHECK(hipGetLastError());
    for (int k = 0; k < 3; ++k) {
      HIP_CHECK(hipEventRecord(ev[0], s));
      for (int i = 0; i < iters; ++i) run((size_t)(i + 1) % copies, 1 << k);
      HIP_CHECK(hipEventRecord(ev[1], s));
      HIP_CHECK(hipGetLastError());
      HIP_CHECK(hipEventSynchronize(ev[1]));
      float ms = 0.0f;
      HIP_CHECK(hipEventElapsedTime(&ms, ev[0], ev[1]));
      ms3[k] = ms / iters;
    }
    int e = 0;
    HIP_CHECK(hipMemcpy(&e, err.p, sizeof(int), hipMemcpyDeviceToHost));
    for (auto &x : ev) (void)hipEventDestroy(x);
    (void)hipStreamDestroy(s);
    if (e) rai::fail(RAI_E_HIP, "attention tile hand-off wait gave up (results discarded)");
  });
}

int rai_w4a8_lane_sums_dev(int32_t *out, const uint8_t *nib, const float *x, size_t rows, size_t cols, size_t m,
                           size_t gs, void *stream) {
  RAI_API_BODY({
    if (!out || !nib || !x) rai::fail(RAI_E_ARG, "null argument");
    if (rows == 0 || cols == 0 || cols % 2 || gs == 0 || gs % 2 || m == 0) rai::fail(RAI_E_SHAPE, "invalid shape");
    hipStream_t s = (hipStream_t)stream;
    const size_t groups = rai::ceil_div(cols, gs);
    rai::DevBuf qn, sc, su;
    qn.alloc(m * cols);
    sc.alloc(m * groups * 4);
    su.alloc(m * groups * 4);
    rai::launch_quantize(x, (int)m, (int)cols, (int)gs, qn.as<int8_t>(), nullptr, sc.as<float>(), su.as<float>(), s);
    rai::launch_lane_sums(out, nib, qn.as<int8_t>(), (int)rows, (int)cols, (int)m, (int)gs, s);
    HIP_CHECK(hipGetLastError());
    HIP_CHECK(hipStreamSynchronize(s));
  });
}

int rai_w4a8_matmul(float *out, const uint8_t *nib, const uint8_t *params, const float *x, size_t rows, size_t cols,
                    size_t m, size_t gs) {
  RAI_API_BODY({
    if (!out || !nib || !params || !x) rai::fail(RAI_E_ARG, "null argument");
    if (rows == 0 || cols == 0 || cols % 2 || gs == 0 || gs % 2 || m == 0) rai::fail(RAI_E_SHAPE, "invalid shape");
    const size_t groups = rai::ceil_div(cols, gs);
    rai::DevBuf dn, dp, dx, dout;
    dn.alloc(rows * cols / 2);
    dp.alloc(rows * groups * 4);
    dx.alloc(m * cols * 4);
    dout.alloc(m * rows * 4);
    HIP_CHECK(hipMemcpy(dn.p, nib, rows * cols / 2, hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(dp.p, params, rows * groups * 4, hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(dx.p, x, m * cols * 4, hipMemcpyHostToDevice));
    const int rc = rai_w4a8_matmul_dev(dout.as<float>(), dn.as<uint8_t>(), dp.as<uint8_t>(), dx.as<float>(), rows,
                                       cols, m, gs, nullptr);
    if (rc != RAI_OK) return rc;
    HIP_CHECK(hipMemcpy(out, dout.p, m * rows * 4, hipMemcpyDeviceToHost));
  });
}

int rai_tied_lm_head_dev(float *logits, const float *hidden, const uint8_t *codes, const uint8_t *params,
                         size_t vocab, size_t n, size_t gs, void *stream) {
  RAI_API_BODY({
    if (!logits || !hidden || !codes || !params) rai::fail(RAI_E_ARG, "null argument");
    if (gs == 0) rai::fail(RAI_E_SHAPE, "group_size must be non-zero");
    if (n == 0 || n % 2) rai::fail(RAI_E_SHAPE, "hidden_size must be non-zero and even");
    hipStream_t s = (hipStream_t)stream;
    const size_t groups = rai::ceil_div(n, gs);
    rai::DevBuf hq, sc, su;
    hq.alloc(n);
    sc.alloc(groups * 4);
    su.alloc(groups * 4);
    rai::launch_tied_lm_head(logits, hidden, codes, params, (int)vocab, (int)n, (int)gs, 1, hq.as<int8_t>(),
                             sc.as<float>(), su.as<float>(), s);
    HIP_CHECK(hipGetLastError());
    HIP_CHECK(hipStreamSynchronize(s));
  });
}

int rai_embed_lookup_dev(float *out, size_t token, const uint8_t *codes, const uint8_t *params, size_t vocab,
                         size_t hidden, size_t gs, void *stream) {
  RAI_API_BODY({
    if (!out || !codes || !params) rai::fail(RAI_E_ARG, "null argument");
    if (gs == 0) rai::fail(RAI_E_SHAPE, "group_size must be non-zero");
    if (token >= vocab) rai::fail(RAI_E_RANGE, "token id is out of range");
    hipStream_t s = (hipStream_t)stream;
    rai::DevBuf tok, err;
    tok.alloc(4);
    err.alloc(4);
    const uint32_t t = (uint32_t)token;
    HIP_CHECK(hipMemcpyAsync(tok.p, &t, 4, hipMemcpyHostToDevice, s));
    HIP_CHECK(hipMemsetAsync(err.p, 0, 4, s));
    rai::launch_embed(tok.as<uint32_t>(), nullptr, 0, 0, 1, codes, params, (int)vocab, (int)hidden, (int)gs, 1.0f,
                      out, err.as<int>(), s);
    HIP_CHECK(hipGetLastError());
    HIP_CHECK(hipStreamSynchronize(s));
  });
}

int rai_argmax_dev(const float *logits, size_t rows, size_t vocab, uint32_t *out, void *stream) {
  RAI_API_BODY({
    if (!logits || !out) rai::fail(RAI_E_ARG, "null argument");
    if (rows == 0 || vocab == 0) rai::fail(RAI_E_SHAPE, "argmax over an empty row");
    if (rows > INT32_MAX || vocab > INT32_MAX) rai::fail(RAI_E_SHAPE, "dimensions overflow");
    launch_argmax(logits, (int)rows, (int)vocab, out, (hipStream_t)stream);
    HIP_CHECK(hipGetLastError());
    HIP_CHECK(hipStreamSynchronize((hipStream_t)stream));
  });
}

int rai_rms_norm_dev(float *out, const float *x, const float *w, size_t m, size_t n, float eps, void *stream) {
  RAI_API_BODY({
    if (!out || !x || !w) rai::fail(RAI_E_ARG, "null argument");
    if (n == 0 || m == 0) rai::fail(RAI_E_SHAPE, "RMSNorm input must not be empty");
    if (!std::isfinite(eps) || eps <= 0.0f) rai::fail(RAI_E_ARG, "RMSNorm epsilon must be finite and positive");
    rai::launch_rmsnorm(x, w, out, nullptr, (int)m, (int)n, eps, (hipStream_t)stream);
    HIP_CHECK(hipGetLastError());
  });
}

int rai_silu_mul_dev(float *gate, const float *up, size_t m, size_t n, void *stream) {
  RAI_API_BODY({
    if (!gate || !up) rai::fail(RAI_E_ARG, "null argument");
    if (n == 0 || m == 0) return RAI_OK;
    rai::launch_silu_mul(gate, up, (int)m, (int)n, (hipStream_t)stream);
    HIP_CHECK(hipGetLastError());
  });
}

int rai_rope_apply_dev(float *heads, size_t nh, size_t hd, const float *c, const float *s, void *stream) {
  RAI_API_BODY({
    if (!heads || !c || !s) rai::fail(RAI_E_ARG, "null argument");
    if (hd == 0 || hd % 2) rai::fail(RAI_E_SHAPE, "RoPE head_dim must be positive and even");
    rai::launch_rope_apply(heads, (int)nh, (int)hd, c, s, (hipStream_t)stream);
    HIP_CHECK(hipGetLastError());
  });
}

int rai_attention_head_dev(float *out, const float *q, const float *k, const float *v, size_t pos, size_t hd,
                           float scale, void *stream) {
  RAI_API_BODY({
    if (!out || !q || !k || !v) rai::fail(RAI_E_ARG, "null argument");
    if (hd == 0 || hd % 8 || hd > 256) rai::fail(RAI_E_SHAPE, "head_dim must be a multiple of 8 up to 256");
    // One head: q [hd], cache rows [pos+1][hd] viewed as one kv head with cap = pos+1.
    rai::DevBuf scores;
    scores.alloc(sizeof(float) * rai::attention_scores_floats(1, 1, (int)(pos + 1)));
    rai::launch_attention(q, (int)hd, k, v, (int)(pos + 1), 0, (int)pos, 1, 1, 1, (int)hd, scale, out, scores.as<float>(),
                          (hipStream_t)stream);
    HIP_CHECK(hipGetLastError());
    HIP_CHECK(hipStreamSynchronize((hipStream_t)stream));
  });
}

int rai_find_ngram_draft(const uint32_t *tokens, size_t len, size_t min_ngram, size_t max_ngram, size_t max_draft,
                         rai_lookup_match *out, int *found) {
  RAI_API_BODY({
    if (!out || !found || (len && !tokens)) rai::fail(RAI_E_ARG, "null argument");
    *found = 0;
    if (max_draft == 0 || len < 2) return RAI_OK;
    if (len > INT32_MAX) rai::fail(RAI_E_SHAPE, "context too long");
    rai::DevBuf dt, dr;
    dt.alloc(len * 4);
    dr.alloc(16);
    HIP_CHECK(hipMemcpy(dt.p, tokens, len * 4, hipMemcpyHostToDevice));
    const int mx = (int)std::min<size_t>(max_ngram, INT32_MAX), mn = (int)std::min<size_t>(min_ngram, INT32_MAX);
    rai::launch_ngram(dt.as<uint32_t>(), (int)len, mn, mx, (int)std::min<size_t>(max_draft, INT32_MAX),
                      dr.as<int>(), nullptr);
    int r[3];
    HIP_CHECK(hipMemcpy(r, dr.p, sizeof(r), hipMemcpyDeviceToHost));
    if (r[0]) {
      *found = 1;
      out->ngram = r[0];
      out->start = r[1];
      out->len = r[2];
    }
  });
}

int rai_lookup_create(rai_model *m, size_t max_ctx, rai_lookup **out) {
  RAI_API_BODY({
    if (!m || !out) rai::fail(RAI_E_ARG, "null argument");
    auto d = std::make_unique<rai_lookup>();
    d->model = m;
    d->max_ctx = std::min<size_t>(max_ctx, m->cfg.max_context);
    if (d->max_ctx == 0) rai::fail(RAI_E_ARG, "prompt-lookup context must be non-zero");
    rai::kv_init(d->kv, *m, d->max_ctx);
    d->ws.init(*m, rai::kChunk, 64);
    d->ctx.alloc((d->max_ctx + 64) * sizeof(uint32_t));
    d->ctx_host.assign(d->max_ctx + 64, 0);
    d->res.alloc(64);
    d->step.alloc(64);
    HIP_CHECK(hipHostMalloc((void **)&d->pin, 4096, hipHostMallocDefault));
    HIP_CHECK(hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking));
    // Step graphs for dense models (the MoE block synchronises with the
    // host to group tokens by expert, which a graph cannot hold).
    const char *env = std::getenv("RAI_STEP_GRAPHS");
    d->graphs = (m->cfg.num_experts == 0 || rai::moe_on_device(*m)) && !(env && env[0] == '0');
    const size_t spans = (size_t)rai::attn_span_index((int)d->max_ctx) + 1;
    d->graph.assign(3 * (rai::kAttnTokens + 1) * spans, nullptr);
    d->graph_uses.assign(3 * (rai::kAttnTokens + 1) * spans, 0);
    d->rng.alloc(sizeof(rai::RngState));
    d->probs.alloc(sizeof(float) * 64 * (size_t)m->cfg.vocab_size);
    d->pscratch.alloc(sizeof(float) * (size_t)m->cfg.vocab_size);
    d->flags.alloc(sizeof(uint32_t) * (size_t)m->cfg.vocab_size);
    HIP_CHECK(hipMemset(d->flags.p, 0, sizeof(uint32_t) * (size_t)m->cfg.vocab_size));
    rai::RngState r;
    rai::rng_seed_from_u64(r, 0);
    HIP_CHECK(hipMemcpy(d->rng.p, &r, sizeof(r), hipMemcpyHostToDevice));
    *out = d.release();
  });
}

void rai_lookup_free(rai_lookup *d) { delete d; }

int rai_lookup_seed(rai_lookup *d, uint64_t seed) {
  RAI_API_BODY({
    if (!d) rai::fail(RAI_E_ARG, "null argument");
    rai::RngState r;
    rai::rng_seed_from_u64(r, seed);
    HIP_CHECK(hipStreamSynchronize(d->stream));
    HIP_CHECK(hipMemcpy(d->rng.p, &r, sizeof(r), hipMemcpyHostToDevice));
  });
}

int rai_std_rng_draws(uint64_t seed, const int *kinds, size_t n, uint64_t *out) {
  RAI_API_BODY({
    if ((!kinds || !out) && n) rai::fail(RAI_E_ARG, "null argument");
    for (size_t i = 0; i < n; ++i)
      if (kinds[i] < 0 || kinds[i] > 3) rai::fail(RAI_E_ARG, "draw kind must be 0..3");
    rai::RngState r;
    rai::rng_seed_from_u64(r, seed);
    DevBuf dr, dk, dout;
    dr.alloc(sizeof(r));
    dk.alloc(sizeof(int) * (n + 1));
    dout.alloc(sizeof(uint64_t) * (n + 1));
    HIP_CHECK(hipMemcpy(dr.p, &r, sizeof(r), hipMemcpyHostToDevice));
    if (n) HIP_CHECK(hipMemcpy(dk.p, kinds, sizeof(int) * n, hipMemcpyHostToDevice));
    rai::launch_rng_draws(dr.as<rai::RngState>(), dk.as<int>(), (int)n, dout.as<uint64_t>(), nullptr);
    HIP_CHECK(hipGetLastError());
    if (n) HIP_CHECK(hipMemcpy(out, dout.p, sizeof(uint64_t) * n, hipMemcpyDeviceToHost));
  });
}

int rai_lookup_kv(rai_lookup *d, rai_kv **out) {
  RAI_API_BODY({
    if (!d || !out) rai::fail(RAI_E_ARG, "null argument");
    *out = &d->kv;
  });
}

int rai_lookup_prefill(rai_lookup *d, const uint32_t *prompt, size_t n, size_t *pos_out) {
  RAI_API_BODY({
    if (!d || !pos_out || (n && !prompt)) rai::fail(RAI_E_ARG, "null argument");
    rai::lookup_prefill(*d, prompt, n, *pos_out);
  });
}

int rai_lookup_step(rai_lookup *d, size_t pos, const uint32_t *context, size_t len, const rai_lookup_config *cfg,
                    uint32_t *out_tokens, size_t out_cap, rai_lookup_metrics *metrics) {
  RAI_API_BODY({
    if (!d || !cfg || !out_tokens || !metrics || (len && !context)) rai::fail(RAI_E_ARG, "null argument");
    rai::lookup_step(*d, pos, context, len, *cfg, out_tokens, out_cap, *metrics);
  });
}

namespace rai {

// The decode loop of `rai run --lookup-k` (cli/run.rs:517-633) after the
// prefill: steps from (pos, context) until max_tokens are generated or the
// window is full.  Fills the step counters and decode_seconds of `s`.
static size_t lookup_decode_loop(rai_lookup &d, const uint32_t *context, size_t len, size_t pos, size_t max_tokens,
                                 const rai_lookup_config &cfg, uint32_t *out, rai_generate_stats &s) {
  auto t1 = std::chrono::steady_clock::now();
  std::vector<uint32_t> ctx(context, context + len);
  ctx.reserve(len + max_tokens + cfg.max_draft + 1);
  std::vector<uint32_t> step_out(cfg.max_draft + 1);
  size_t gen = 0;
  while (gen < max_tokens && pos < d.max_ctx) {
    rai_lookup_metrics met{};
    lookup_step(d, pos, ctx.data(), ctx.size(), cfg, step_out.data(), step_out.size(), met);
    for (size_t i = 0; i < met.produced; ++i) {
      out[gen++] = step_out[i];
      ctx.push_back(step_out[i]);
    }
    pos += met.produced;
    s.steps++;
    if (met.drafted) s.steps_with_draft++;
    s.drafted += met.drafted;
    s.accepted += met.accepted;
  }
  s.generated = gen;
  s.decode_seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t1).count();
  return gen;
}

}  // namespace rai

int rai_lookup_generate(rai_lookup *d, const uint32_t *prompt, size_t n, size_t max_tokens,
                        const rai_lookup_config *cfg, uint32_t *out, size_t out_cap, size_t *n_out,
                        rai_generate_stats *st) {
  RAI_API_BODY({
    if (!d || !prompt || !cfg || !out || !n_out) rai::fail(RAI_E_ARG, "null argument");
    if (out_cap < max_tokens + cfg->max_draft) rai::fail(RAI_E_SHAPE, "output buffer too small");
    rai_generate_stats s{};
    s.prompt_tokens = n;
    auto t0 = std::chrono::steady_clock::now();
    size_t pos = 0;
    rai::lookup_prefill(*d, prompt, n, pos);
    s.prefill_seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    *n_out = rai::lookup_decode_loop(*d, prompt, n, pos, max_tokens, *cfg, out, s);
    if (st) *st = s;
  });
}

int rai_lookup_decode(rai_lookup *d, const uint32_t *context, size_t len, size_t pos, size_t max_tokens,
                      const rai_lookup_config *cfg, uint32_t *out, size_t out_cap, size_t *n_out,
                      rai_generate_stats *st) {
  RAI_API_BODY({
    if (!d || !context || !cfg || !out || !n_out) rai::fail(RAI_E_ARG, "null argument");
    if (out_cap < max_tokens + cfg->max_draft) rai::fail(RAI_E_SHAPE, "output buffer too small");
    if (len == 0 || pos + 1 != len) rai::fail(RAI_E_ARG, "context[len - 1] must be the token at pos");
    rai_generate_stats s{};
    s.prompt_tokens = len;
    *n_out = rai::lookup_decode_loop(*d, context, len, pos, max_tokens, *cfg, out, s);
    if (st) *st = s;
  });
}

int rai_kv_export(const rai_kv *kv, size_t layer, int which, float *out, size_t npos) {
  RAI_API_BODY({
    if (!kv || !out) rai::fail(RAI_E_ARG, "null argument");
    if (layer >= (size_t)kv->layers) rai::fail(RAI_E_ARG, "layer index out of range");
    if (npos > kv->filled[layer])
      rai::fail(RAI_E_WATERMARK, "KV export above the watermark (filled " + std::to_string(kv->filled[layer]) + ")");
    HIP_CHECK(hipDeviceSynchronize());  // as rai_kv_read
    const size_t hd = kv->hd;
    if (which == 0) {
      for (int h = 0; h < kv->nkv; ++h)
        HIP_CHECK(hipMemcpy(out + (size_t)h * npos * hd, kv->kc((int)layer) + (size_t)h * kv->cap * hd,
                            sizeof(float) * npos * hd, hipMemcpyDeviceToHost));
    } else {
      // d-major V [head][hd][vstride]: copy [hd][npos] and transpose.
      std::vector<float> tmp(hd * npos);
      for (int h = 0; h < kv->nkv; ++h) {
        if (npos)
          HIP_CHECK(hipMemcpy2D(tmp.data(), npos * sizeof(float), kv->vc((int)layer) + (size_t)h * hd * kv->vstride,
                                kv->vstride * sizeof(float), npos * sizeof(float), hd, hipMemcpyDeviceToHost));
        float *dst = out + (size_t)h * npos * hd;
        for (size_t d = 0; d < hd; ++d)
          for (size_t p = 0; p < npos; ++p) dst[p * hd + d] = tmp[d * npos + p];
      }
    }
  });
}

int rai_kv_import(rai_kv *kv, size_t layer, int which, const float *rows, size_t npos) {
  RAI_API_BODY({
    if (!kv || !rows) rai::fail(RAI_E_ARG, "null argument");
    if (layer >= (size_t)kv->layers) rai::fail(RAI_E_ARG, "layer index out of range");
    if (which != 0 && which != 1) rai::fail(RAI_E_ARG, "which must be 0 (K) or 1 (V)");
    if (npos > kv->cap) rai::fail(RAI_E_RANGE, "KV cache position is out of range");
    const size_t hd = kv->hd;
    HIP_CHECK(hipDeviceSynchronize());  // no decoder work may still use the rows
    if (which == 0) {
      for (int h = 0; h < kv->nkv; ++h)
        if (npos)
          HIP_CHECK(hipMemcpy(kv->kc((int)layer) + (size_t)h * kv->cap * hd, rows + (size_t)h * npos * hd,
                              sizeof(float) * npos * hd, hipMemcpyHostToDevice));
    } else {
      // d-major V [head][hd][vstride]: transpose to [hd][npos], then copy.
      std::vector<float> tmp(hd * npos);
      for (int h = 0; h < kv->nkv; ++h) {
        const float *src = rows + (size_t)h * npos * hd;
        for (size_t p = 0; p < npos; ++p)
          for (size_t d = 0; d < hd; ++d) tmp[d * npos + p] = src[p * hd + d];
        if (npos)
          HIP_CHECK(hipMemcpy2D(kv->vc((int)layer) + (size_t)h * hd * kv->vstride, kv->vstride * sizeof(float),
                                tmp.data(), npos * sizeof(float), npos * sizeof(float), hd, hipMemcpyHostToDevice));
      }
    }
    kv->filled[layer] = npos;
  });
}

namespace rai {

// The plain decode loop from a prefilled state (context[len - 1] is the
// token at pos): decode_one per token (lookup.rs:428-455), the token by
// argmax (sampler = null: run.rs:692-735 at temperature 0 without a
// repetition penalty) or by the repetition penalty and sample_token with
// the sampler's config (run.rs:720-721).
static void greedy_decode(rai_lookup &d, const uint32_t *context, size_t len, size_t pos, size_t steps,
                          uint32_t *out, const rai_sampler_config *sampler = nullptr) {
  const rai_lookup_config plain{1, 1, 1, 0.0f};  // search parameters unused (no search)
  std::vector<uint32_t> ctx(context, context + len);
  ctx.reserve(len + steps);
  uint32_t tok[2];
  for (size_t i = 0; i < steps; ++i) {
    if (pos >= d.max_ctx) fail(RAI_E_RANGE, "generation exceeds the context window");
    rai_lookup_metrics met{};
    lookup_step(d, pos, ctx.data(), ctx.size(), plain, tok, 2, met, false, sampler);
    out[i] = tok[0];
    ctx.push_back(tok[0]);
    ++pos;
  }
}

}  // namespace rai

int rai_greedy_generate(rai_lookup *d, const uint32_t *prompt, size_t n, size_t steps, uint32_t *out) {
  RAI_API_BODY({
    if (!d || !prompt || !out) rai::fail(RAI_E_ARG, "null argument");
    size_t pos = 0;
    rai::lookup_prefill(*d, prompt, n, pos);
    rai::greedy_decode(*d, prompt, n, pos, steps, out);
  });
}

int rai_greedy_decode(rai_lookup *d, const uint32_t *context, size_t len, size_t pos, size_t steps, uint32_t *out) {
  RAI_API_BODY({
    if (!d || !context || !out) rai::fail(RAI_E_ARG, "null argument");
    if (len == 0 || pos + 1 != len) rai::fail(RAI_E_ARG, "context[len - 1] must be the token at pos");
    rai::greedy_decode(*d, context, len, pos, steps, out);
  });
}

int rai_sample_decode(rai_lookup *d, const uint32_t *context, size_t len, size_t pos, size_t steps,
                      const rai_sampler_config *cfg, uint32_t *out) {
  RAI_API_BODY({
    if (!d || !context || !cfg || !out) rai::fail(RAI_E_ARG, "null argument");
    if (len == 0 || pos + 1 != len) rai::fail(RAI_E_ARG, "context[len - 1] must be the token at pos");
    rai::greedy_decode(*d, context, len, pos, steps, out, cfg);
  });
}

int rai_sample_tokens(const float *logits, size_t vocab, const uint32_t *recent, size_t n_recent,
                      const rai_sampler_config *cfg, uint64_t seed, size_t draws, uint32_t *out) {
  RAI_API_BODY({
    if (!logits || !cfg || !out || (n_recent && !recent)) rai::fail(RAI_E_ARG, "null argument");
    if (vocab == 0 || vocab > INT32_MAX || n_recent > INT32_MAX) rai::fail(RAI_E_SHAPE, "invalid vocabulary size");
    hipStream_t s;
    HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    rai::DevBuf dl, dc, dw, df, dr, dout;
    dl.alloc(sizeof(float) * vocab);
    dc.alloc(sizeof(uint32_t) * (n_recent + 1));
    dw.alloc(sizeof(float) * vocab);
    df.alloc(sizeof(uint32_t) * vocab);
    dr.alloc(sizeof(rai::RngState));
    dout.alloc(sizeof(uint32_t) * std::max<size_t>(draws, 1));
    rai::RngState r;
    rai::rng_seed_from_u64(r, seed);
    HIP_CHECK(hipMemcpyAsync(dl.p, logits, sizeof(float) * vocab, hipMemcpyHostToDevice, s));
    if (n_recent) HIP_CHECK(hipMemcpyAsync(dc.p, recent, sizeof(uint32_t) * n_recent, hipMemcpyHostToDevice, s));
    HIP_CHECK(hipMemcpyAsync(dr.p, &r, sizeof(r), hipMemcpyHostToDevice, s));
    HIP_CHECK(hipMemsetAsync(df.p, 0, sizeof(uint32_t) * vocab, s));
    const int top_k = (int)std::min<size_t>(cfg->top_k, INT32_MAX);
    for (size_t i = 0; i < draws; ++i)
      rai::launch_sample_plain(dl.as<float>(), (int)vocab, dc.as<uint32_t>(), (int)n_recent, cfg->temperature, top_k,
                               cfg->top_p, cfg->repetition_penalty, dr.as<rai::RngState>(), dw.as<float>(),
                               df.as<uint32_t>(), dout.as<uint32_t>() + i, nullptr, s);
    HIP_CHECK(hipGetLastError());
    if (draws) HIP_CHECK(hipMemcpyAsync(out, dout.p, sizeof(uint32_t) * draws, hipMemcpyDeviceToHost, s));
    HIP_CHECK(hipStreamSynchronize(s));
    HIP_CHECK(hipStreamDestroy(s));
  });
}

// ------------------------------------------------ speculative decoder --

struct rai_spec {
  rai_model *draft = nullptr, *target = nullptr;
  rai_kv dkv, tkv;
  size_t max_ctx = 0;
  rai::Workspace dws, tws;
  DevBuf prompt;  // prompt tokens for the prefill
  DevBuf toks;    // [last, drafts (<= 63), produced (<= 64)]
  DevBuf dlog, dprobs, tprobs, scratch, rng, res;
  int *pin = nullptr;  // pinned: res (2 ints) then the produced tokens
  hipStream_t stream = nullptr;
  ~rai_spec() {
    if (pin) (void)hipHostFree(pin);
    if (stream) (void)hipStreamDestroy(stream);
  }
};

namespace rai {

// One decode step of model `md` at `pos` on the token at dev_tok: embed,
// forward (watermark checks and commit), logits into w.logits row 0.
static void decode_on(rai_model &md, rai_kv &kv, Workspace &w, const uint32_t *dev_tok, size_t pos, hipStream_t s) {
  forward_check(md, kv, w, 1, pos);
  launch_embed(dev_tok, nullptr, 0, 0, 1, md.emb_codes, md.emb_params, md.cfg.vocab_size, md.cfg.hidden_size,
               md.cfg.embed_group_size, md.cfg.embed_scale, w.hid.as<float>(), w.err.as<int>(), s);
  forward_enqueue(md, kv, w, 1, pos, s, nullptr);
  forward_commit(kv, 1, pos);
}

// SpeculativeDecoder::step (speculative.rs:180-391): k draft decode steps
// (each token sampled, or taken by argmax in the greedy variant), one
// batched target forward over [last, drafts], then acceptance, the draft
// model's catch-up on its last token when every draft was accepted, and
// both watermarks truncated to pos + produced.
static void spec_step(rai_spec &d, size_t pos, uint32_t last, const rai_spec_config &cfg, uint32_t *out,
                      size_t cap, rai_spec_metrics &met) {
  rai_model &dm = *d.draft, &tm = *d.target;
  const int V = tm.cfg.vocab_size;
  if (cfg.draft_k == 0) fail(RAI_E_ARG, "speculative draft_k must be non-zero");
  if (cfg.draft_k > 63) fail(RAI_E_ARG, "draft_k above 63 is not supported");
  if (!std::isfinite(cfg.temperature)) fail(RAI_E_ARG, "temperature must be finite");
  if (pos >= d.max_ctx) fail(RAI_E_RANGE, "decode position exceeds the speculative context window");
  if (cap < cfg.draft_k + 1) fail(RAI_E_SHAPE, "output buffer must hold draft_k + 1 tokens");
  check_tokens(tm, &last, 1);
  const bool sampled = cfg.temperature > 1e-6f;
  const float T = cfg.temperature;
  const int k = (int)std::min<size_t>(cfg.draft_k, d.max_ctx - pos - 1);
  hipStream_t s = d.stream;
  uint32_t *toks = d.toks.as<uint32_t>();
  int *res = d.res.as<int>();
  HIP_CHECK(hipGetLastError());
  d.pin[64] = (int)last;
  HIP_CHECK(hipMemcpyAsync(toks, d.pin + 64, sizeof(uint32_t), hipMemcpyHostToDevice, s));
  if (k == 0) {
    decode_on(tm, d.tkv, d.tws, toks, pos, s);
    logits(tm, d.tws, 1, s);
    if (sampled) {
      launch_spec_sample(d.tws.logits.as<float>(), d.tprobs.as<float>(), nullptr, nullptr, V, toks, 0, T,
                         d.rng.as<RngState>(), d.scratch.as<float>(), res, s);
    } else {
      launch_argmax(d.tws.logits.as<float>(), 1, V, d.tws.am.as<uint32_t>(), s);
      launch_accept(d.tws.am.as<uint32_t>(), toks, 1, 1, 0, res, s, nullptr);
    }
  } else {
    for (int i = 0; i < k; ++i) {
      decode_on(dm, d.dkv, d.dws, toks + i, pos + i, s);
      logits(dm, d.dws, 1, s);
      if (sampled)
        launch_draw(d.dws.logits.as<float>(), V, T, d.rng.as<RngState>(), d.dlog.as<float>() + (size_t)i * V,
                    d.scratch.as<float>(), toks + i + 1, s);
      else
        launch_argmax(d.dws.logits.as<float>(), 1, V, toks + i + 1, s);
    }
    const int m = k + 1;
    forward_check(tm, d.tkv, d.tws, m, pos);
    launch_embed(toks, nullptr, 0, 0, m, tm.emb_codes, tm.emb_params, V, tm.cfg.hidden_size, tm.cfg.embed_group_size,
                 tm.cfg.embed_scale, d.tws.hid.as<float>(), d.tws.err.as<int>(), s);
    forward_enqueue(tm, d.tkv, d.tws, m, pos, s, nullptr);
    forward_commit(d.tkv, m, pos);
    logits(tm, d.tws, m, s);
    if (sampled) {
      launch_spec_sample(d.tws.logits.as<float>(), d.tprobs.as<float>(), d.dlog.as<float>(), d.dprobs.as<float>(),
                         V, toks, k, T, d.rng.as<RngState>(), d.scratch.as<float>(), res, s);
    } else {
      launch_argmax(d.tws.logits.as<float>(), m, V, d.tws.am.as<uint32_t>(), s);
      launch_accept(d.tws.am.as<uint32_t>(), toks, m, 1, k, res, s, nullptr);
    }
  }
  HIP_CHECK(hipGetLastError());
  HIP_CHECK(hipMemcpyAsync(d.pin, res, 2 * sizeof(int), hipMemcpyDeviceToHost, s));
  HIP_CHECK(hipMemcpyAsync(d.pin + 2, toks + k + 1, (size_t)(k + 1) * sizeof(uint32_t), hipMemcpyDeviceToHost, s));
  int e[2] = {0, 0}, f[2] = {0, 0};
  HIP_CHECK(hipMemcpyAsync(e, d.tws.err.p, sizeof(e), hipMemcpyDeviceToHost, s));
  HIP_CHECK(hipMemcpyAsync(f, d.dws.err.p, sizeof(f), hipMemcpyDeviceToHost, s));
  HIP_CHECK(hipStreamSynchronize(s));
  if (e[0] || e[1] || f[0] || f[1]) {
    for (auto &x : d.dkv.filled) x = std::min(x, pos);
    for (auto &x : d.tkv.filled) x = std::min(x, pos);
    raise_kernel_errors(d.dws, s, f);
    raise_kernel_errors(d.tws, s, e);
  }
  const int acc = d.pin[0], prod = d.pin[1];
  for (auto &x : d.tkv.filled) x = std::min(x, pos + (size_t)prod);
  if (k > 0 && acc == k) {
    // Every draft accepted: the draft model's catch-up step on its last
    // draft token (row pos + k of the draft cache), finished before the
    // step returns so that the draft cache is whole for a caller that reads
    // it next.  If its attention wait gave up, that row stays above the
    // watermark and the step fails.
    decode_on(dm, d.dkv, d.dws, toks + k, pos + k, s);
    HIP_CHECK(hipGetLastError());
    HIP_CHECK(hipMemcpyAsync(f, d.dws.err.p, sizeof(f), hipMemcpyDeviceToHost, s));
    HIP_CHECK(hipStreamSynchronize(s));
    if (f[0] || f[1]) {
      for (auto &x : d.dkv.filled) x = std::min(x, pos + (size_t)k);
      raise_kernel_errors(d.dws, s, f);
    }
  }
  for (auto &x : d.dkv.filled) x = std::min(x, pos + (size_t)prod);
  for (int i = 0; i < prod; ++i) out[i] = (uint32_t)d.pin[2 + i];
  met.accepted = (size_t)acc;
  met.drafted = (size_t)k;
  met.produced = (size_t)prod;
  met.accept_rate = k ? (float)acc / (float)k : 0.0f;
}

}  // namespace rai

int rai_spec_create(rai_model *draft, rai_model *target, size_t max_ctx, rai_spec **out) {
  RAI_API_BODY({
    if (!draft || !target || !out) rai::fail(RAI_E_ARG, "null argument");
    if (draft->cfg.vocab_size != target->cfg.vocab_size)
      rai::fail(RAI_E_ARG, "draft and target vocabularies differ; speculative decoding needs one tokenizer");
    auto d = std::make_unique<rai_spec>();
    d->draft = draft;
    d->target = target;
    const size_t dctx = std::min<size_t>(max_ctx, draft->cfg.max_context);
    const size_t tctx = std::min<size_t>(max_ctx, target->cfg.max_context);
    d->max_ctx = std::min(dctx, tctx);
    if (d->max_ctx == 0) rai::fail(RAI_E_ARG, "speculative decoding context must be non-zero");
    rai::kv_init(d->dkv, *draft, dctx);
    rai::kv_init(d->tkv, *target, tctx);
    d->dws.init(*draft, rai::kChunk, 64);
    d->tws.init(*target, rai::kChunk, 64);
    const size_t V = target->cfg.vocab_size;
    d->prompt.alloc(d->max_ctx * sizeof(uint32_t));
    d->toks.alloc(160 * sizeof(uint32_t));
    d->dlog.alloc(sizeof(float) * 64 * V);
    d->dprobs.alloc(sizeof(float) * 64 * V);
    d->tprobs.alloc(sizeof(float) * 65 * V);
    d->scratch.alloc(sizeof(float) * V);
    d->res.alloc(64);
    d->rng.alloc(sizeof(rai::RngState));
    rai::RngState r;
    rai::rng_seed_from_u64(r, 0);
    HIP_CHECK(hipMemcpy(d->rng.p, &r, sizeof(r), hipMemcpyHostToDevice));
    HIP_CHECK(hipHostMalloc((void **)&d->pin, 4096, hipHostMallocDefault));
    HIP_CHECK(hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking));
    *out = d.release();
  });
}

void rai_spec_free(rai_spec *d) { delete d; }

int rai_spec_kv(rai_spec *d, int which, rai_kv **out) {
  RAI_API_BODY({
    if (!d || !out) rai::fail(RAI_E_ARG, "null argument");
    if (which != 0 && which != 1) rai::fail(RAI_E_ARG, "which must be 0 (draft) or 1 (target)");
    *out = which ? &d->tkv : &d->dkv;
  });
}

int rai_spec_seed(rai_spec *d, uint64_t seed) {
  RAI_API_BODY({
    if (!d) rai::fail(RAI_E_ARG, "null argument");
    rai::RngState r;
    rai::rng_seed_from_u64(r, seed);
    HIP_CHECK(hipStreamSynchronize(d->stream));
    HIP_CHECK(hipMemcpy(d->rng.p, &r, sizeof(r), hipMemcpyHostToDevice));
  });
}

int rai_spec_prefill(rai_spec *d, const uint32_t *prompt, size_t n, size_t *pos_out) {
  RAI_API_BODY({
    if (!d || !prompt || !pos_out) rai::fail(RAI_E_ARG, "null argument");
    if (n == 0) rai::fail(RAI_E_ARG, "prompt must contain at least one token");
    if (n > d->max_ctx) rai::fail(RAI_E_RANGE, "prompt exceeds the speculative context window");
    rai::check_tokens(*d->target, prompt, n);
    HIP_CHECK(hipMemcpyAsync(d->prompt.p, prompt, n * sizeof(uint32_t), hipMemcpyHostToDevice, d->stream));
    const size_t cnt = n - 1;
    for (int which = 0; which < 2; ++which) {
      rai_model &md = which ? *d->target : *d->draft;
      rai_kv &kv = which ? d->tkv : d->dkv;
      rai::Workspace &w = which ? d->tws : d->dws;
      for (size_t p = 0; p < cnt; p += rai::kChunk) {
        const int m = (int)std::min<size_t>(rai::kChunk, cnt - p);
        launch_embed(d->prompt.as<uint32_t>() + p, nullptr, 0, 0, m, md.emb_codes, md.emb_params,
                     md.cfg.vocab_size, md.cfg.hidden_size, md.cfg.embed_group_size, md.cfg.embed_scale,
                     w.hid.as<float>(), w.err.as<int>(), d->stream);
        rai::forward(md, kv, w, m, p, d->stream);
      }
      try {
        rai::check_kernel_error(w, d->stream);
      } catch (...) {
        for (auto &f : kv.filled) f = 0;
        throw;
      }
    }
    *pos_out = cnt;
  });
}

int rai_spec_step(rai_spec *d, size_t pos, uint32_t last_token, const rai_spec_config *cfg, uint32_t *out_tokens,
                  size_t out_cap, rai_spec_metrics *metrics) {
  RAI_API_BODY({
    if (!d || !cfg || !out_tokens || !metrics) rai::fail(RAI_E_ARG, "null argument");
    rai::spec_step(*d, pos, last_token, *cfg, out_tokens, out_cap, *metrics);
  });
}

int rai_debug_set_attention_spin(int polls) { RAI_API_BODY(rai::set_attention_spin(polls)); }

int rai_dev_malloc(size_t bytes, void **out) {
  RAI_API_BODY({
    if (!out) rai::fail(RAI_E_ARG, "null argument");
    HIP_CHECK(hipMalloc(out, bytes ? bytes : 1));
  });
}
int rai_dev_free(void *p) { RAI_API_BODY(HIP_CHECK(hipFree(p))); }
int rai_memcpy_h2d(void *dst, const void *src, size_t n) {
  RAI_API_BODY(HIP_CHECK(hipMemcpy(dst, src, n, hipMemcpyHostToDevice)));
}
int rai_memcpy_d2h(void *dst, const void *src, size_t n) {
  RAI_API_BODY(HIP_CHECK(hipMemcpy(dst, src, n, hipMemcpyDeviceToHost)));
}
int rai_device_synchronize(void) { RAI_API_BODY(HIP_CHECK(hipDeviceSynchronize())); }
int rai_stream_create(void **out) {
  RAI_API_BODY({
    hipStream_t s;
    HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *out = s;
  });
}
int rai_stream_destroy(void *s) { RAI_API_BODY(HIP_CHECK(hipStreamDestroy((hipStream_t)s))); }
int rai_event_create(void **out) {
  RAI_API_BODY({
    hipEvent_t e;
    HIP_CHECK(hipEventCreate(&e));
    *out = e;
  });
}
int rai_event_destroy(void *e) { RAI_API_BODY(HIP_CHECK(hipEventDestroy((hipEvent_t)e))); }
int rai_event_record(void *e, void *s) { RAI_API_BODY(HIP_CHECK(hipEventRecord((hipEvent_t)e, (hipStream_t)s))); }
int rai_event_elapsed_ms(void *a, void *b, float *ms) {
  RAI_API_BODY(HIP_CHECK(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b)));
}
int rai_stream_synchronize(void *s) { RAI_API_BODY(HIP_CHECK(hipStreamSynchronize((hipStream_t)s))); }

}  // extern "C"
