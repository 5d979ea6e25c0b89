// Test infrastructure (not part of the product): relay's own Engine -- continuous batching,
// chunked prefill, prefix caching, preemption (engine/src/engine.cpp) -- built from the
// reference's sources by oracle/Makefile, driving this build's HIP backend compiled against
// relay's own headers (engine/include/relay/*.h plus the HipOptions block INTEGRATION.md
// adds), beside relay's CPU backend (engine/src/cpu_backend.cpp) on the same requests.
//
//   relay_engine_hip MODEL NUM_BLOCKS BLOCK_SIZE MAX_BATCH_TOKENS MAX_SEQS PREFIX_CACHING REQUESTS SEED
//
// MODEL: a Hugging Face model directory (relay's HostWeights::load), or
//   synthetic:hidden,intermediate,layers,heads,kv_heads,head_dim,vocab,bias
//   (weights N(0, 0.02) from a seeded generator, rounded to fp16 values so that both backends
//   compute with the same numbers; norms 1).
// REQUESTS: comma-separated prompt_len:max_new[:shared_prefix_len] (prompts of seeded random
//   ids; requests that give a shared prefix length start with the same ids).
// Prints one JSON line: the greedy tokens of both runs equal or not, the worst per-row relative
// logit difference (relay's test_reference metric: max|a-b| / max|b|), the engine's counters.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <memory>
#include <sstream>
#include <string>
#include <utility>
#include <vector>

#include "relay/backend.h"
#include "relay/engine.h"
#include "relay/safetensors.h"
#include "relay/weights.h"

namespace {

std::uint64_t splitmix(std::uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// Standard normal draw i of stream s (Box-Muller on two splitmix uniforms).
float normal(std::uint64_t seed, std::uint64_t s, std::uint64_t i) {
  const std::uint64_t a = splitmix(seed ^ splitmix(s * 0x100000001B3ull + 2 * i));
  const std::uint64_t b = splitmix(seed ^ splitmix(s * 0x100000001B3ull + 2 * i + 1));
  const double u1 = (static_cast<double>(a >> 11) + 1.0) / 9007199254740993.0;
  const double u2 = static_cast<double>(b >> 11) / 9007199254740992.0;
  return static_cast<float>(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
}

void fill(std::vector<float>& v, std::size_t n, std::uint64_t seed, std::uint64_t s, float std) {
  v.resize(n);
  for (std::size_t i = 0; i < n; ++i) v[i] = relay::f16_to_f32(relay::f32_to_f16(std * normal(seed, s, i)));
}

relay::HostWeights synthetic(const std::string& spec, std::uint64_t seed) {
  std::vector<int> f;
  std::stringstream ss(spec);
  for (std::string x; std::getline(ss, x, ',');) f.push_back(std::atoi(x.c_str()));
  if (f.size() != 8) throw std::invalid_argument("synthetic:hidden,intermediate,layers,heads,kv_heads,head_dim,vocab,bias");
  relay::HostWeights w;
  relay::ModelConfig& c = w.config;
  c.model_type = f[7] ? "qwen2" : "llama";
  c.hidden = f[0];
  c.intermediate = f[1];
  c.layers = f[2];
  c.heads = f[3];
  c.kv_heads = f[4];
  c.head_dim = f[5];
  c.vocab = f[6];
  c.qkv_bias = f[7] != 0;
  c.tie_embeddings = true;
  c.max_position = 1 << 16;
  const std::size_t H = c.hidden, Q = c.q_dim(), KV = c.kv_dim(), I = c.intermediate, V = c.vocab;
  std::uint64_t s = 0;
  fill(w.embed, V * H, seed, s++, 0.02f);
  w.final_norm.assign(H, 1.0f);
  for (int l = 0; l < c.layers; ++l) {
    relay::LayerWeights L;
    L.attn_norm.assign(H, 1.0f);
    L.mlp_norm.assign(H, 1.0f);
    fill(L.wqkv, (Q + 2 * KV) * H, seed, s++, 0.02f);
    if (c.qkv_bias) fill(L.bqkv, Q + 2 * KV, seed, s++, 0.02f);
    fill(L.wo, H * Q, seed, s++, 0.02f);
    fill(L.w_gate_up, 2 * I * H, seed, s++, 0.02f);
    fill(L.w_down, H * I, seed, s++, 0.02f);
    w.layers.push_back(std::move(L));
  }
  return w;
}

struct Run {
  std::map<std::uint64_t, std::vector<int>> tokens;
  std::map<std::pair<std::uint64_t, int>, std::vector<float>> logits;
  relay::EngineStats stats;
};

Run run(relay::Backend& be, const std::vector<relay::Request>& reqs, const relay::EngineOptions& opt, int vocab) {
  Run r;
  relay::Engine eng(be, opt);
  eng.on_logits = [&](std::uint64_t id, int index, const float* lg) {
    r.logits[{id, index}] = std::vector<float>(lg, lg + vocab);
  };
  for (const auto& q : reqs) eng.add(q);
  r.tokens = eng.run_all();
  r.stats = eng.stats();
  return r;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 9) {
    std::fprintf(stderr,
                 "usage: %s MODEL NUM_BLOCKS BLOCK_SIZE MAX_BATCH_TOKENS MAX_SEQS PREFIX_CACHING REQUESTS SEED\n",
                 argv[0]);
    return 2;
  }
  try {
    const std::string model = argv[1];
    const int num_blocks = std::atoi(argv[2]), block_size = std::atoi(argv[3]);
    const int max_batch_tokens = std::atoi(argv[4]), max_seqs = std::atoi(argv[5]);
    const bool prefix = std::atoi(argv[6]) != 0;
    const std::uint64_t seed = std::strtoull(argv[8], nullptr, 10);
    const relay::HostWeights w =
        model.rfind("synthetic:", 0) == 0 ? synthetic(model.substr(10), seed) : relay::HostWeights::load(model);
    const int vocab = w.config.vocab;

    std::vector<relay::Request> reqs;
    std::vector<int> shared;
    std::stringstream ss(argv[7]);
    std::uint64_t id = 1;
    for (std::string item; std::getline(ss, item, ',');) {
      int len = 0, max_new = 0, pre = 0;
      if (std::sscanf(item.c_str(), "%d:%d:%d", &len, &max_new, &pre) < 2) throw std::invalid_argument("bad request " + item);
      relay::Request q;
      q.id = id;
      for (int i = 0; i < len; ++i) {
        if (i < pre) {
          while (static_cast<int>(shared.size()) <= i) shared.push_back(static_cast<int>(splitmix(seed * 7919 + shared.size()) % vocab));
          q.prompt.push_back(shared[i]);
        } else {
          q.prompt.push_back(static_cast<int>(splitmix(seed * 104729 + id * 65537 + i) % vocab));
        }
      }
      q.params.max_new_tokens = max_new;
      q.params.ignore_eos = true;
      reqs.push_back(std::move(q));
      ++id;
    }
    relay::EngineOptions opt;
    opt.max_batch_tokens = max_batch_tokens;
    opt.max_seqs = max_seqs;
    opt.prefix_caching = prefix;

    auto cpu = relay::make_cpu_backend(w, num_blocks, block_size);
    relay::HipOptions ho;  // the fast kernels, fp16 weights
    auto hip = relay::make_hip_backend(w, num_blocks, block_size, 0, max_batch_tokens, num_blocks * block_size, ho);
    const Run a = run(*cpu, reqs, opt, vocab);
    const Run b = run(*hip, reqs, opt, vocab);

    double worst = 0;
    int rows = 0;
    for (const auto& [key, la] : a.logits) {
      auto it = b.logits.find(key);
      if (it == b.logits.end()) continue;
      const auto& lb = it->second;
      double num = 0, den = 1e-6;
      for (int i = 0; i < vocab; ++i) {
        num = std::max(num, std::fabs(static_cast<double>(lb[i]) - la[i]));
        den = std::max(den, std::fabs(static_cast<double>(la[i])));
      }
      worst = std::max(worst, num / den);
      ++rows;
    }
    std::printf(
        "{\"backend\": \"%s\", \"tokens_equal\": %s, \"requests\": %zu, \"rows\": %d, \"worst_rel\": %.3e, "
        "\"steps\": [%llu, %llu], \"preemptions\": [%llu, %llu], \"prefix_hit_tokens\": [%llu, %llu]}\n",
        hip->name().c_str(), a.tokens == b.tokens ? "true" : "false", reqs.size(), rows, worst,
        static_cast<unsigned long long>(a.stats.steps), static_cast<unsigned long long>(b.stats.steps),
        static_cast<unsigned long long>(a.stats.preemptions), static_cast<unsigned long long>(b.stats.preemptions),
        static_cast<unsigned long long>(a.stats.prefix_hit_tokens),
        static_cast<unsigned long long>(b.stats.prefix_hit_tokens));
    return 0;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "error: %s\n", e.what());
    return 1;
  }
}
