// rai-run: the `rai run` generate loop (rai-infer/src/cli/run.rs:242-633)
// over the C ABI, for a .raimodel on one GPU.  Token ids in, token ids out
// (the tokenizer and chat templates sit outside this path).
//
//   rai-run MODEL --prompt-ids 1,2,3 [--max-tokens 64] [--temperature 0.7]
//           [--top-k 40] [--top-p 0.9] [--repetition-penalty 1.1]
//           [--seed 42] [--max-context N] [--eos ID] [--max-groups G] [--verbose]
//           [--lookup-k K --lookup-ngram 3 --lookup-min-ngram 1]
//           [--draft DRAFT.raimodel --draft-k 6]
//
// Modes as run.rs: --draft (draft-model speculation) and --lookup-k
// (prompt lookup) are mutually exclusive and need --top-k 0 --top-p 1
// --repetition-penalty 1; without either, plain decoding, each token by the
// repetition penalty over the context and sample_token (sampler.rs:47-199).
// One deliberate extension: the reference refuses the speculative modes at
// --temperature <= 1e-6 (run.rs:205-213); here they select greedy
// acceptance, whose tokens equal plain greedy decoding.  Generated ids go to
// stdout, one line; the statistics to stderr.
#include <cfloat>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "rai_hip.h"

namespace {

struct Args {
  std::string model, draft;
  std::vector<uint32_t> prompt;
  size_t max_tokens = 64, max_context = 0, draft_k = 6, lookup_k = 0, lookup_ngram = 3, lookup_min_ngram = 1;
  float temperature = 0.7f, top_p = 0.9f, repetition_penalty = 1.1f;  // run.rs:40-56
  size_t top_k = 40;
  uint64_t seed = 42;
  long eos = -1;
  int max_groups = 0;  // 0: the reference's MAX_GROUPS (gemm.rs:1167)
  bool verbose = false;
};

[[noreturn]] void die(const std::string &msg) {
  std::fprintf(stderr, "rai-run: %s\n", msg.c_str());
  std::exit(2);
}

void check(int rc, const char *what) {
  if (rc != RAI_OK) die(std::string(what) + ": " + rai_last_error());
}

std::vector<uint32_t> parse_ids(const char *s) {
  std::vector<uint32_t> out;
  const char *p = s;
  while (*p) {
    char *end = nullptr;
    const unsigned long v = std::strtoul(p, &end, 10);
    if (end == p) die(std::string("bad token id list: ") + s);
    out.push_back((uint32_t)v);
    p = end;
    while (*p == ',' || *p == ' ') ++p;
  }
  return out;
}

Args parse(int argc, char **argv) {
  Args a;
  for (int i = 1; i < argc; ++i) {
    const std::string k = argv[i];
    auto val = [&]() -> const char * {
      if (i + 1 >= argc) die("missing value for " + k);
      return argv[++i];
    };
    if (k == "--prompt-ids") a.prompt = parse_ids(val());
    else if (k == "--max-tokens") a.max_tokens = std::strtoull(val(), nullptr, 10);
    else if (k == "--temperature") a.temperature = std::strtof(val(), nullptr);
    else if (k == "--top-k") a.top_k = std::strtoull(val(), nullptr, 10);
    else if (k == "--top-p") a.top_p = std::strtof(val(), nullptr);
    else if (k == "--repetition-penalty") a.repetition_penalty = std::strtof(val(), nullptr);
    else if (k == "--seed") a.seed = std::strtoull(val(), nullptr, 10);
    else if (k == "--max-context") a.max_context = std::strtoull(val(), nullptr, 10);
    else if (k == "--eos") a.eos = std::strtol(val(), nullptr, 10);
    else if (k == "--draft") a.draft = val();
    else if (k == "--draft-k") a.draft_k = std::strtoull(val(), nullptr, 10);
    else if (k == "--lookup-k") a.lookup_k = std::strtoull(val(), nullptr, 10);
    else if (k == "--lookup-ngram") a.lookup_ngram = std::strtoull(val(), nullptr, 10);
    else if (k == "--lookup-min-ngram") a.lookup_min_ngram = std::strtoull(val(), nullptr, 10);
    else if (k == "--max-groups") a.max_groups = (int)std::strtol(val(), nullptr, 10);
    else if (k == "--verbose") a.verbose = true;
    else if (!k.empty() && k[0] != '-' && a.model.empty()) a.model = k;
    else die("unknown argument " + k);
  }
  // validate_args (run.rs:134-215), for the options this driver takes.
  if (a.model.empty()) die("a MODEL path is required");
  if (a.prompt.empty()) die("--prompt-ids must not be empty");
  if (a.max_tokens == 0) die("--max-tokens must be greater than zero");
  if (!(std::isfinite(a.temperature) && a.temperature >= 0.0f && a.temperature <= 2.0f))
    die("--temperature must be within [0, 2]");
  if (!(std::isfinite(a.top_p) && a.top_p >= FLT_MIN && a.top_p <= 1.0f)) die("--top-p must be within (0, 1]");
  if (!(std::isfinite(a.repetition_penalty) && a.repetition_penalty >= 0.01f && a.repetition_penalty <= 4.0f))
    die("--repetition-penalty must be within [0.01, 4]");
  if (!a.draft.empty() && a.lookup_k > 0) die("--draft and --lookup-k are mutually exclusive");
  // MAX_SPECULATIVE_TOKENS = 32, MAX_LOOKUP_NGRAM = 16 (run.rs:25-29).
  if (!a.draft.empty() && (a.draft_k < 1 || a.draft_k > 32)) die("--draft-k must be between 1 and 32");
  if (a.lookup_k > 32) die("--lookup-k must be between 1 and 32");
  if (a.lookup_k > 0 && (a.lookup_ngram < 1 || a.lookup_ngram > 16))
    die("--lookup-ngram must be between 1 and 16");
  if (a.lookup_k > 0 && (a.lookup_min_ngram < 1 || a.lookup_min_ngram > a.lookup_ngram))
    die("--lookup-min-ngram must be between 1 and --lookup-ngram");
  // Verification compares against the exact sampled distribution.
  if ((!a.draft.empty() || a.lookup_k > 0) &&
      !(a.top_k == 0 && a.top_p == 1.0f && std::fabs(a.repetition_penalty - 1.0f) < FLT_EPSILON))
    die("speculative decoding requires --top-k 0, --top-p 1 and --repetition-penalty 1");
  return a;
}

double ms_since(std::chrono::steady_clock::time_point t) {
  return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t).count();
}

}  // namespace

int main(int argc, char **argv) {
  const Args a = parse(argc, argv);
  rai_model *model = nullptr;
  check(rai_model_open(a.model.c_str(), a.max_groups, &model), "loading the model");
  rai_model_config cfg{};
  check(rai_model_get_config(model, &cfg), "reading the model config");
  const size_t max_ctx = a.max_context ? std::min<size_t>(a.max_context, cfg.max_context) : cfg.max_context;
  if (a.prompt.size() > max_ctx) die("prompt exceeds the context window");
  std::vector<uint32_t> all(a.prompt);
  size_t generated = 0;
  auto emit = [&](const uint32_t *t, size_t n, size_t &pos) {
    bool eos = false;
    const size_t remaining = std::min(max_ctx - pos, a.max_tokens - generated);
    for (size_t i = 0; i < n && i < remaining; ++i) {
      if (a.eos >= 0 && t[i] == (uint32_t)a.eos) {
        eos = true;
        break;
      }
      all.push_back(t[i]);
      ++pos;
      if (++generated >= a.max_tokens) break;
    }
    return eos;
  };

  if (!a.draft.empty()) {
    rai_model *draft = nullptr;
    check(rai_model_open(a.draft.c_str(), a.max_groups, &draft), "loading the draft model");
    rai_spec *dec = nullptr;
    check(rai_spec_create(draft, model, max_ctx, &dec), "creating the speculative decoder");
    check(rai_spec_seed(dec, a.seed), "seeding");
    const auto t0 = std::chrono::steady_clock::now();
    size_t pos = 0;
    check(rai_spec_prefill(dec, a.prompt.data(), a.prompt.size(), &pos), "prefill");
    std::fprintf(stderr, "\nPrefill: %zu tokens in %.1fms\n", a.prompt.size(), ms_since(t0));
    const auto t1 = std::chrono::steady_clock::now();
    const rai_spec_config sc{a.draft_k, a.temperature};
    std::vector<uint32_t> out(a.draft_k + 1);
    size_t drafted = 0, accepted = 0;
    while (generated < a.max_tokens && pos < max_ctx) {
      rai_spec_metrics m{};
      check(rai_spec_step(dec, pos, all.back(), &sc, out.data(), out.size(), &m), "speculative step");
      if (m.produced == 0) die("speculative decoder made no progress");
      drafted += m.drafted;
      accepted += m.accepted;
      if (a.verbose) std::fprintf(stderr, "[spec:%zud/%zua]", m.drafted, m.accepted);
      if (emit(out.data(), m.produced, pos)) break;
    }
    const double ms = ms_since(t1);
    std::fprintf(stderr, "\n--- Speculative Stats ---\nTokens: %zu, %.2f tok/s\n", generated, generated / (ms / 1e3));
    std::fprintf(stderr, "Drafted: %zu, Accepted: %zu, Rate: %.1f%%\n", drafted, accepted,
                 drafted ? 100.0 * accepted / drafted : 0.0);
    rai_spec_free(dec);
    rai_model_free(draft);
  } else if (a.lookup_k > 0) {
    rai_lookup *dec = nullptr;
    check(rai_lookup_create(model, max_ctx, &dec), "creating the prompt-lookup decoder");
    check(rai_lookup_seed(dec, a.seed), "seeding");
    std::fprintf(stderr, "Prompt-lookup: K=%zu, n-gram %zu..%zu (draft copied from context, no draft model)\n",
                 a.lookup_k, a.lookup_ngram, a.lookup_min_ngram);
    const auto t0 = std::chrono::steady_clock::now();
    size_t pos = 0;
    check(rai_lookup_prefill(dec, a.prompt.data(), a.prompt.size(), &pos), "prefill");
    const double pms = ms_since(t0);
    std::fprintf(stderr, "\nPrefill: %zu tokens in %.1fms (%.1f tok/s)\n", a.prompt.size(), pms,
                 a.prompt.size() / (pms / 1e3));
    const rai_lookup_config lc{a.lookup_k, a.lookup_ngram, a.lookup_min_ngram, a.temperature};
    std::vector<uint32_t> out(a.lookup_k + 1);
    size_t drafted = 0, accepted = 0, steps = 0, with_draft = 0;
    const auto t1 = std::chrono::steady_clock::now();
    while (generated < a.max_tokens && pos < max_ctx) {
      if (pos + 1 != all.size()) die("prompt-lookup context and decode position went out of sync");
      rai_lookup_metrics m{};
      check(rai_lookup_step(dec, pos, all.data(), all.size(), &lc, out.data(), out.size(), &m), "lookup step");
      if (m.produced == 0) die("prompt-lookup decoder made no progress");
      ++steps;
      drafted += m.drafted;
      accepted += m.accepted;
      with_draft += m.matched_ngram != 0;
      if (a.verbose) std::fprintf(stderr, "[lookup:%zud/%zua/n%zu]", m.drafted, m.accepted, m.matched_ngram);
      if (emit(out.data(), m.produced, pos)) break;
    }
    const double ms = ms_since(t1);
    std::fprintf(stderr, "\n--- Prompt-Lookup Stats ---\nTokens: %zu, %.2f tok/s\n", generated, generated / (ms / 1e3));
    std::fprintf(stderr, "Drafted: %zu, Accepted: %zu, Rate: %.1f%%\n", drafted, accepted,
                 drafted ? 100.0 * accepted / drafted : 0.0);
    std::fprintf(stderr, "Steps: %zu (%zu with a draft, %.1f%%), %.2f tokens/step\n", steps, with_draft,
                 100.0 * with_draft / (steps ? steps : 1), (double)generated / (steps ? steps : 1));
    rai_lookup_free(dec);
  } else {
    // Prefill of the first N - 1 tokens, then one decode step per token, each
    // token by the repetition penalty and sample_token (run.rs:640-735).
    rai_lookup *dec = nullptr;
    check(rai_lookup_create(model, max_ctx, &dec), "creating the decoder");
    check(rai_lookup_seed(dec, a.seed), "seeding");
    const auto t0 = std::chrono::steady_clock::now();
    size_t pos = 0;
    check(rai_lookup_prefill(dec, a.prompt.data(), a.prompt.size(), &pos), "prefill");
    const double pms = ms_since(t0);
    std::fprintf(stderr, "\nPrefill: %zu tokens in %.1fms (%.1f tok/s)\n", a.prompt.size(), pms,
                 a.prompt.size() / (pms / 1e3));
    const size_t steps = std::min(a.max_tokens, max_ctx - pos);
    std::vector<uint32_t> out(steps);
    const auto t1 = std::chrono::steady_clock::now();
    const rai_sampler_config sc{a.temperature, a.top_k, a.top_p, a.repetition_penalty};
    check(rai_sample_decode(dec, a.prompt.data(), a.prompt.size(), pos, steps, &sc, out.data()), "decoding");
    const double ms = ms_since(t1);
    emit(out.data(), out.size(), pos);
    std::fprintf(stderr, "\n--- Stats ---\nTokens: %zu, %.2f tok/s\n", generated, generated / (ms / 1e3));
    rai_lookup_free(dec);
  }
  for (size_t i = a.prompt.size(); i < all.size(); ++i)
    std::printf("%s%u", i == a.prompt.size() ? "" : ",", all[i]);
  std::printf("\n");
  rai_model_free(model);
  return 0;
}
