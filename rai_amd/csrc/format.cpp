// .raimodel validation and views (rai-infer/src/format.rs), host side.
#include "format.h"

#include <cmath>
#include <cstring>

namespace rai {

namespace {

constexpr size_t kHeaderV1 = 64;
constexpr size_t kHeaderV2 = 128;
constexpr uint32_t kMaxHidden = 65536, kMaxInter = 1048576, kMaxLayers = 1024, kMaxHeads = 1024;
constexpr uint32_t kMaxVocab = 10000000, kMaxContext = 1000000;
constexpr int kRefMaxGroups = 128;                           // gemm.rs:1167
constexpr size_t kMaxRopeTableBytes = 512ull * 1024 * 1024;  // layers.rs:21-27

uint32_t rd32(const uint8_t *p) {
  uint32_t v;
  std::memcpy(&v, p, 4);
  return v;
}
uint64_t rd64(const uint8_t *p) {
  uint64_t v;
  std::memcpy(&v, p, 8);
  return v;
}
float rdf(const uint8_t *p) {
  float v;
  std::memcpy(&v, p, 4);
  return v;
}

[[noreturn]] void bad(const std::string &m) { fail(RAI_E_FORMAT, m); }

// read_linear (format.rs:487-530).
LinearView read_linear(const uint8_t *data, size_t sec_off, size_t sec_len, size_t &off,
                       uint32_t rows, uint32_t cols, uint32_t gs, const std::string &label) {
  const size_t hdr_end = checked_add(off, 8, "linear header end");
  if (hdr_end > sec_len) bad(label + ": linear header truncated");
  const uint32_t r = rd32(data + sec_off + off), c = rd32(data + sec_off + off + 4);
  if (r != rows || c != cols)
    bad(label + ": linear is [" + std::to_string(r) + ", " + std::to_string(c) + "], expected [" +
        std::to_string(rows) + ", " + std::to_string(cols) + "]");
  const size_t groups = ceil_div(cols, gs);
  const size_t pbytes = checked_mul(checked_mul(rows, groups, "linear parameter groups"), 4,
                                    "linear parameter bytes");
  const size_t nbytes = (checked_mul(rows, cols, "linear elements") + 1) / 2;
  const size_t p_end = checked_add(hdr_end, pbytes, "linear parameter end");
  const size_t end = checked_add(p_end, nbytes, "linear data end");
  if (end > sec_len) bad(label + ": linear data truncated");
  LinearView v;
  v.rows = rows;
  v.cols = cols;
  v.group_size = gs;
  v.params_off = sec_off + hdr_end;
  v.params_len = pbytes;
  v.nib_off = sec_off + p_end;
  v.nib_len = nbytes;
  off = end;
  return v;
}

// validate_group_params (format.rs:1492-1504).
void check_params(const uint8_t *p, size_t len, const std::string &label) {
  if (len % 4) bad(label + " quantization parameters are misaligned");
  for (size_t i = 0; i < len / 4; ++i) {
    uint16_t sb, zb;
    std::memcpy(&sb, p + i * 4, 2);
    std::memcpy(&zb, p + i * 4 + 2, 2);
    const float s = f16_bits_to_f32(sb), z = f16_bits_to_f32(zb);
    if (!std::isfinite(s) || s <= 0.0f || !std::isfinite(z))
      bad(label + " quantization group " + std::to_string(i) +
          " contains an invalid scale or zero point");
  }
}

// validate_f32_vector (format.rs:1510-1521).
void check_f32(const uint8_t *p, size_t n, const std::string &label) {
  for (size_t i = 0; i < n; ++i)
    if (!std::isfinite(rdf(p + i * 4)))
      bad(label + " weight " + std::to_string(i) + " is non-finite");
}

// read_optional_positive (format.rs:1368-1374).
float optional_positive(const uint8_t *d, size_t off, const char *name) {
  const float v = rdf(d + off);
  if (!std::isfinite(v) || v < 0.0f)
    bad(std::string(name) + " must be finite and non-negative (0.0 disables it)");
  return v;
}

}  // namespace

float f16_bits_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {  // subnormal: renormalise
      int e = -1;
      do {
        ++e;
        man <<= 1;
      } while ((man & 0x400u) == 0);
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3FFu) << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7F800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

ModelView parse_model(const uint8_t *d, size_t n, int max_groups) {
  ModelView mv;
  rai_model_config &c = mv.cfg;
  // parse_header (format.rs:1098-1183)
  if (n < kHeaderV1) bad("file too small for header: " + std::to_string(n) + " bytes");
  if (std::memcmp(d, "RAIM", 4) != 0) bad("not a .raimodel file: expected magic \"RAIM\"");
  c.version = rd32(d + 4);
  if (c.version != 1 && c.version != 2)
    bad("unsupported format version: " + std::to_string(c.version));
  mv.header_size = c.version == 1 ? kHeaderV1 : kHeaderV2;
  if (n < mv.header_size) bad("file too small for a v2 header");
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
  const uint8_t bits = d[48], embed_bits = d[50];
  c.group_size = d[49];
  c.embed_group_size = d[51];
  c.embed_scale = 1.0f;
  float attn_scale = 0.0f;
  if (c.version == 2) {
    // read_v2_capabilities (format.rs:1192-1365).  Malformed blocks are
    // format errors; well-formed capabilities this build does not run
    // (activations other than SiLU, biases, QK/sandwich/post norms, llama3
    // RoPE, softcaps, per-layer RoPE) are refused as unsupported, never
    // ignored.
    for (int i = 56; i < 64; ++i)
      if (d[i]) bad("header bytes 56..64 are reserved and must be zero");
    for (int i = 109; i < 128; ++i)
      if (d[i]) bad("header bytes 109..128 are reserved and must be zero");
    if (d[64] > 1) bad("unsupported activation code " + std::to_string(d[64]));
    const uint8_t flags = d[65], rope_type = d[66], bias_mask = d[67];
    if (flags & ~0x1Fu) bad("header flags set bits this reader does not implement");
    if (bias_mask & ~0x7Fu) bad("bias_mask sets bits beyond the 7 projections");
    if (((flags & 1) != 0) != (bias_mask != 0)) bad("header is inconsistent: bias flag vs bias_mask");
    if ((flags & 0x02) && (flags & 0x08)) bad("header sets both per-head and full-width QK norm");
    if ((flags & 0x04) && (flags & 0x10)) bad("header sets both sandwich norms and post-norm");
    if (rope_type > 1) bad("unsupported rope_type " + std::to_string(rope_type));
    if (rope_type == 0) {
      for (int i = 68; i < 84; ++i)
        if (d[i]) bad("rope_type 0 (default) must leave the RoPE scaling parameters zero");
    }
    const float es = rdf(d + 84);
    if (!std::isfinite(es) || es <= 0.0f) bad("embed_scale must be finite and positive");
    c.embed_scale = es;
    const float attn_cap = optional_positive(d, 88, "attn_logit_softcap");
    const float final_cap = optional_positive(d, 92, "final_logit_softcap");
    attn_scale = optional_positive(d, 96, "attn_scale");
    uint16_t ne;
    std::memcpy(&ne, d + 105, 2);
    c.num_experts = ne;
    c.experts_per_token = d[107];
    const uint8_t moe_flags = d[108];
    if (moe_flags & ~1u) bad("moe_flags sets bits this reader does not implement");
    c.norm_topk_prob = moe_flags & 1;
    if (c.num_experts == 0) {
      if (c.experts_per_token != 0 || moe_flags != 0)
        bad("header declares no experts but sets experts_per_token or moe_flags");
    } else {
      if (c.num_experts < 2) bad("a dense MLP is stored with num_experts = 0");
      if (c.experts_per_token == 0 || c.experts_per_token > c.num_experts)
        bad("experts_per_token is out of range");
    }
    const float local_theta = optional_positive(d, 100, "rope_local_theta");
    const uint8_t stride = d[104];
    if ((local_theta > 0.0f) != (stride > 0)) bad("per-layer RoPE needs both fields or neither");
    if (stride == 1) bad("global_layer_stride of 1 makes every layer global");
    if (d[64] != 0) fail(RAI_E_UNSUPPORTED, "GeLU-tanh (GeGLU) models are not supported");
    if (flags != 0) fail(RAI_E_UNSUPPORTED, "bias / QK-norm / sandwich / post-norm layers are not supported");
    if (rope_type != 0) fail(RAI_E_UNSUPPORTED, "llama3 RoPE scaling is not supported");
    if (attn_cap != 0.0f || final_cap != 0.0f) fail(RAI_E_UNSUPPORTED, "logit softcaps are not supported");
    if (stride != 0) fail(RAI_E_UNSUPPORTED, "per-layer RoPE bases are not supported");
  }
  // validate_config (format.rs:1376-1480).
  const struct {
    const char *name;
    uint32_t v, mx;
  } lims[] = {{"hidden_size", c.hidden_size, kMaxHidden},   {"num_layers", c.num_layers, kMaxLayers},
              {"num_heads", c.num_heads, kMaxHeads},         {"num_kv_heads", c.num_kv_heads, kMaxHeads},
              {"head_dim", c.head_dim, kMaxHidden},          {"intermediate_size", c.intermediate_size, kMaxInter},
              {"vocab_size", c.vocab_size, kMaxVocab},       {"max_context", c.max_context, kMaxContext}};
  for (auto &l : lims)
    if (l.v == 0 || l.v > l.mx) bad(std::string("invalid ") + l.name + ": " + std::to_string(l.v));
  if (bits != 4) bad("unsupported weight bit width " + std::to_string(bits) + "; expected 4");
  if (embed_bits != 8) bad("unsupported embedding bit width " + std::to_string(embed_bits) + "; expected 8");
  if (c.group_size == 0 || c.embed_group_size == 0) bad("quantization group sizes must be non-zero");
  if (c.group_size % 2 || c.embed_group_size % 2) bad("quantization group sizes must be even");
  if (c.hidden_size % 2 || c.intermediate_size % 2)
    bad("hidden and intermediate dimensions must be even for packed 4-bit kernels");
  if (c.head_dim % 8) bad("head_dim must be a multiple of 8 for SIMD attention kernels");
  if (c.num_heads % c.num_kv_heads) bad("num_heads must be divisible by num_kv_heads");
  const size_t attn_dim = (size_t)c.num_heads * c.head_dim;
  if (attn_dim > kMaxInter) bad("num_heads * head_dim is too large");
  if (attn_dim % 2) bad("num_heads * head_dim must be even for packed 4-bit kernels");
  const int limit = max_groups > 0 ? max_groups : kRefMaxGroups;
  const size_t gs = c.group_size;
  const size_t mg = std::max(std::max(ceil_div(c.hidden_size, gs), ceil_div(c.intermediate_size, gs)),
                             ceil_div(attn_dim, gs));
  if (mg > (size_t)limit)
    bad("model requires " + std::to_string(mg) + " quantization groups; kernel maximum is " +
        std::to_string(limit));
  if (ceil_div(c.hidden_size, c.embed_group_size) > (size_t)limit)
    bad("embedding requires too many quantization groups");
  if (!std::isfinite(c.rope_theta) || c.rope_theta <= 0.0f) bad("rope_theta must be finite and positive");
  if (!std::isfinite(c.norm_eps) || c.norm_eps <= 0.0f) bad("norm_eps must be finite and positive");
  const size_t rope_bytes = checked_mul(checked_mul((size_t)c.max_context, c.head_dim / 2, "RoPE elements"), 8,
                                        "RoPE table bytes");
  if (rope_bytes > kMaxRopeTableBytes) bad("RoPE table exceeds its 512 MiB budget");
  const size_t ns = rd32(d + 52);
  const size_t tied_ns = (size_t)c.num_layers + 2, untied_ns = (size_t)c.num_layers + 3;
  if (ns != tied_ns && ns != untied_ns) bad("invalid section count " + std::to_string(ns));
  mv.tied = ns == tied_ns;
  c.tied = mv.tied;
  // Section table (format.rs:587-628).
  const size_t tab_end = checked_add(mv.header_size, checked_mul(ns, 16, "section table size"),
                                     "section table end");
  if (n < tab_end) bad("file too small for section table");
  size_t prev = tab_end;
  mv.sections.resize(ns);
  for (size_t i = 0; i < ns; ++i) {
    const uint64_t o = rd64(d + mv.header_size + i * 16), s = rd64(d + mv.header_size + i * 16 + 8);
    if (s == 0) bad("section " + std::to_string(i) + " is empty");
    if (o != prev) bad("section " + std::to_string(i) + " is not contiguous");
    if (o + s < o || o + s > n) bad("section " + std::to_string(i) + " extends beyond file");
    mv.sections[i] = {o, s};
    prev = o + s;
  }
  if (prev != n) bad("unreferenced trailing data");
  // Embedding (format.rs:793-823).
  {
    const size_t eg = ceil_div(c.hidden_size, c.embed_group_size);
    const size_t pb = checked_mul(checked_mul(c.vocab_size, eg, "embedding groups"), 4, "embedding params");
    const size_t db = checked_mul(c.vocab_size, c.hidden_size, "embedding data");
    if (mv.sections[0].second != pb + db) bad("embedding section size mismatch");
    mv.emb_params_off = mv.sections[0].first;
    mv.emb_codes_off = mv.sections[0].first + pb;
    check_params(d + mv.emb_params_off, pb, "embedding");
  }
  // Layers (format.rs:826-1006).
  const uint32_t H = c.hidden_size, F = c.intermediate_size;
  const uint32_t qd = (uint32_t)attn_dim, kvd = c.num_kv_heads * c.head_dim;
  const uint32_t dims[7][2] = {{qd, H}, {kvd, H}, {kvd, H}, {H, qd}, {F, H}, {F, H}, {H, F}};
  static const char *names[7] = {"q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"};
  mv.layers.resize(c.num_layers);
  for (uint32_t li = 0; li < c.num_layers; ++li) {
    const size_t so = mv.sections[1 + li].first, sl = mv.sections[1 + li].second;
    const std::string lab = "layer " + std::to_string(li);
    LayerView &L = mv.layers[li];
    size_t off = 0;
    for (int p = 0; p < 7; ++p) {
      L.lin[p] = read_linear(d, so, sl, off, dims[p][0], dims[p][1], c.group_size, lab);
      check_params(d + L.lin[p].params_off, L.lin[p].params_len, lab + " " + names[p]);
    }
    if (c.num_experts > 0) {
      const size_t rb = checked_mul(checked_mul(c.num_experts, H, "router elements"), 4, "router bytes");
      if (off + rb > sl) bad(lab + ": router truncated");
      L.router_off = so + off;
      check_f32(d + L.router_off, rb / 4, lab + " router");
      off += rb;
      for (uint32_t e = 1; e < c.num_experts; ++e)
        for (int p = 4; p < 7; ++p) {
          LinearView v = read_linear(d, so, sl, off, dims[p][0], dims[p][1], c.group_size,
                                     lab + ": expert " + std::to_string(e) + " " + names[p]);
          check_params(d + v.params_off, v.params_len, lab + " expert " + std::to_string(e));
          L.experts.push_back(v);
        }
    }
    const size_t nb = (size_t)H * 4;
    if (off + 2 * nb != sl) bad(lab + ": section size mismatch");
    L.in_norm_off = so + off;
    L.post_norm_off = so + off + nb;
    check_f32(d + L.in_norm_off, H, lab + " input norm");
    check_f32(d + L.post_norm_off, H, lab + " pre-MLP norm");
  }
  // Final norm and lm_head (format.rs:1012-1082).
  {
    const auto &s = mv.sections[1 + c.num_layers];
    if (s.second != (uint64_t)H * 4) bad("final norm section size mismatch");
    mv.final_norm_off = s.first;
    check_f32(d + s.first, H, "final norm");
  }
  if (!mv.tied) {
    const auto &s = mv.sections[ns - 1];
    size_t off = 0;
    mv.lm_head = read_linear(d, s.first, s.second, off, c.vocab_size, H, c.group_size, "lm_head");
    if (off != s.second) bad("lm_head section size mismatch");
    check_params(d + mv.lm_head.params_off, mv.lm_head.params_len, "lm_head");
  }
  // ModelConfig::attention_scale (format.rs:275-281).
  mv.attention_scale = attn_scale > 0.0f ? attn_scale : 1.0f / std::sqrt((float)c.head_dim);
  c.attn_scale = mv.attention_scale;
  return mv;
}

}  // namespace rai
