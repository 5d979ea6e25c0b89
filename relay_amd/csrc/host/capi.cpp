// The backend half of the C ABI (include/relay_hip.h): relay_hip_backend_* over the C++
// HipBackend, with relay's C-API error convention -- exceptions become a return of -1
// (or NULL) and a per-thread message (c_api.cpp:31-46), here in rh_last_error().
// Also the host-side synthetic-input generator.
#include <cmath>
#include <algorithm>
#include <cstring>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "relay/backend.h"
#include "relay_hip.h"

namespace relay_hip {
void set_error(const std::string& msg);
}

namespace relay {
namespace hip_detail {
Backend* new_backend(const ModelConfig& c, const rh_host_weights* hw, bool synthetic, std::uint64_t seed, float std,
                     int num_blocks, int block_size, int device, int max_tokens, int max_context, HipOptions o);
double last_forward_ms(const Backend* b);
int forward_into(Backend* b, const ForwardBatch& batch, float* dst, std::size_t cap);
void fill_kv_random(Backend* b, std::uint64_t seed, float std);
}  // namespace hip_detail
}  // namespace relay

struct relay_hip_backend {
  relay::Backend* be = nullptr;
};

namespace {

relay::ModelConfig to_config(const rh_model_config& c) {
  relay::ModelConfig m;
  m.model_type = c.qkv_bias ? "qwen2" : "llama";
  m.hidden = c.hidden;
  m.intermediate = c.intermediate;
  m.layers = c.layers;
  m.heads = c.heads;
  m.kv_heads = c.kv_heads;
  m.head_dim = c.head_dim;
  m.vocab = c.vocab;
  m.rms_eps = c.rms_eps;
  m.rope_theta = c.rope_theta;
  m.tie_embeddings = c.tie_embeddings != 0;
  m.qkv_bias = c.qkv_bias != 0;
  if (c.rope_scaling_llama3) {
    m.rope_scaling.type = "llama3";
    m.rope_scaling.factor = c.rope_factor;
    m.rope_scaling.low_freq_factor = c.rope_low_freq_factor;
    m.rope_scaling.high_freq_factor = c.rope_high_freq_factor;
    m.rope_scaling.original_max_position = c.rope_original_max_position;
  }
  return m;
}

relay::HipOptions to_options(const rh_backend_options* o) {
  if (!o) return relay::HipOptions::from_env();
  relay::HipOptions h;
  h.reference_attention = o->reference_attention != 0;
  h.int8_weights = o->int8_weights != 0;
  return h;
}

template <class F>
int guarded(F&& f) {
  try {
    f();
    return 0;
  } catch (const std::exception& e) {
    relay_hip::set_error(e.what());
    return -1;
  }
}

uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

}  // namespace

extern "C" {

rh_backend_options rh_backend_options_from_env(void) {
  relay::HipOptions h = relay::HipOptions::from_env();
  return rh_backend_options{h.reference_attention ? 1 : 0, h.int8_weights ? 1 : 0};
}

relay_hip_backend* relay_hip_backend_new(const rh_model_config* config, const rh_host_weights* weights,
                                         int num_blocks, int block_size, int device, int max_batch_tokens,
                                         int max_context, const rh_backend_options* options) {
  relay_hip_backend* out = nullptr;
  guarded([&] {
    if (!config || !weights) throw std::invalid_argument("config and weights are required");
    auto* b = new relay_hip_backend;
    try {
      b->be = relay::hip_detail::new_backend(to_config(*config), weights, false, 0, 0.0f, num_blocks, block_size,
                                             device, max_batch_tokens, max_context, to_options(options));
    } catch (...) {
      delete b;
      throw;
    }
    out = b;
  });
  return out;
}

relay_hip_backend* relay_hip_backend_new_synthetic(const rh_model_config* config, uint64_t seed, float std,
                                                   int num_blocks, int block_size, int device, int max_batch_tokens,
                                                   int max_context, const rh_backend_options* options) {
  relay_hip_backend* out = nullptr;
  guarded([&] {
    if (!config) throw std::invalid_argument("config is required");
    auto* b = new relay_hip_backend;
    try {
      b->be = relay::hip_detail::new_backend(to_config(*config), nullptr, true, seed, std, num_blocks, block_size,
                                             device, max_batch_tokens, max_context, to_options(options));
    } catch (...) {
      delete b;
      throw;
    }
    out = b;
  });
  return out;
}

void relay_hip_backend_free(relay_hip_backend* b) {
  if (!b) return;
  delete b->be;
  delete b;
}

int relay_hip_backend_forward(relay_hip_backend* b, int n_seqs, const int* n_tokens, const int* tokens,
                              const int* start_pos, const int* table_len, const int* tables, const int* want_logits,
                              int all_logits, float* logits, size_t logits_cap) {
  int rows = -1;
  int rc = guarded([&] {
    if (!b) throw std::invalid_argument("no backend");
    relay::ForwardBatch batch;
    batch.all_logits = all_logits != 0;
    const int* tp = tokens;
    const int* bp = tables;
    for (int s = 0; s < n_seqs; ++s) {
      relay::SeqChunk ch;
      ch.tokens.assign(tp, tp + n_tokens[s]);
      ch.start_pos = start_pos[s];
      ch.block_table.assign(bp, bp + table_len[s]);
      ch.want_logits = want_logits ? want_logits[s] != 0 : true;
      batch.seqs.push_back(std::move(ch));
      tp += n_tokens[s];
      bp += table_len[s];
    }
    // Straight into the caller's buffer (relay's forward() returns a vector, which would be
    // one more copy of every logits row).
    rows = relay::hip_detail::forward_into(b->be, batch, logits, logits_cap);
  });
  return rc ? -1 : rows;
}

size_t relay_hip_backend_kv_block_bytes(const relay_hip_backend* b) { return b ? b->be->kv_block_bytes() : 0; }

int relay_hip_backend_read_kv_block(relay_hip_backend* b, int layer, int block, void* k_out, void* v_out) {
  return guarded([&] { b->be->read_kv_block(layer, block, k_out, v_out); });
}

int relay_hip_backend_write_kv_block(relay_hip_backend* b, int layer, int block, const void* k_in, const void* v_in) {
  return guarded([&] { b->be->write_kv_block(layer, block, k_in, v_in); });
}

int relay_hip_backend_read_kv_layer(relay_hip_backend* b, int layer, const int* blocks, int n, void* out) {
  return guarded([&] { b->be->read_kv_layer(layer, std::vector<int>(blocks, blocks + n), out); });
}

int relay_hip_backend_write_kv_layer(relay_hip_backend* b, int layer, const int* blocks, int n, const void* in) {
  return guarded([&] { b->be->write_kv_layer(layer, std::vector<int>(blocks, blocks + n), in); });
}

int relay_hip_backend_wait_kv_written(relay_hip_backend* b, int layer) {
  return guarded([&] { b->be->wait_kv_written(layer); });
}

int relay_hip_backend_update_weight(relay_hip_backend* b, const char* name, const float* src, size_t n) {
  return guarded([&] { b->be->update_weight(name, src, n); });
}

int relay_hip_backend_fill_kv_random(relay_hip_backend* b, uint64_t seed, float std) {
  return guarded([&] { relay::hip_detail::fill_kv_random(b->be, seed, std); });
}

double relay_hip_backend_last_forward_ms(const relay_hip_backend* b) {
  return b ? relay::hip_detail::last_forward_ms(b->be) : 0.0;
}

// Counter-based normal draws: the uniform pair of element i comes from splitmix64 mixes
// of (key, 2i + 1) and (key, 2i + 2), key = mix(seed, stream); Box-Muller in double.
void rh_synth_normal_f32(float* out, size_t n, uint64_t seed, uint64_t stream_id, float mean, float std) {
  const uint64_t key = mix64(seed + 0x9E3779B97F4A7C15ull * (stream_id + 1));
  auto work = [&](size_t lo, size_t hi) {
    for (size_t i = lo; i < hi; ++i) {
      const uint64_t a = mix64(key + 0x9E3779B97F4A7C15ull * (2 * i + 1));
      const uint64_t b = mix64(key + 0x9E3779B97F4A7C15ull * (2 * i + 2));
      const double u1 = static_cast<double>((a >> 11) + 1) * (1.0 / 9007199254740992.0);
      const double u2 = static_cast<double>(b >> 11) * (1.0 / 9007199254740992.0);
      const double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586476925286766559 * u2);
      out[i] = static_cast<float>(mean + std * z);
    }
  };
  const size_t threads = n < (1u << 16) ? 1 : std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  std::vector<std::thread> pool;
  for (size_t t = 0; t < threads; ++t) pool.emplace_back(work, n * t / threads, n * (t + 1) / threads);
  for (auto& th : pool) th.join();
}

}  // extern "C"
