// TEST INFRASTRUCTURE ONLY. A C interface over the reference's own CPU backend and
// engine, compiled from the sources in /root/reference by oracle/Makefile into
// oracle/_ref/librelay_ref.so. It exists to pin the oracle (cpu_oracle.cpp) bit for bit
// and to write the golden vectors under tests/golden/; nothing in relay_amd uses it.
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "relay/backend.h"
#include "relay/engine.h"
#include "relay/safetensors.h"
#include "relay/sampler.h"

namespace {
thread_local std::string g_error;

struct Handle {
  relay::HostWeights w;
  std::unique_ptr<relay::Backend> be;
};
}  // namespace

extern "C" {

const char* ref_last_error(void) { return g_error.c_str(); }

// Loads a Hugging Face model directory with the reference loader and builds its CPU backend.
void* ref_model_load(const char* dir, int num_blocks, int block_size) {
  try {
    auto* h = new Handle();
    h->w = relay::HostWeights::load(dir);
    h->be = relay::make_cpu_backend(h->w, num_blocks, block_size);
    return h;
  } catch (const std::exception& e) {
    g_error = e.what();
    return nullptr;
  }
}

void ref_model_free(void* h) { delete static_cast<Handle*>(h); }

int ref_model_vocab(void* h) { return static_cast<Handle*>(h)->w.config.vocab; }

int ref_forward(void* hp, int n_seqs, const int* n_tokens, const int* tokens, const int* start_pos,
                const int* table_len, const int* tables, const int* want_logits, int all_logits, float* logits,
                size_t cap) {
  auto* h = static_cast<Handle*>(hp);
  try {
    relay::ForwardBatch b;
    b.all_logits = all_logits != 0;
    const int* tp = tokens;
    const int* bp = tables;
    for (int s = 0; s < n_seqs; ++s) {
      relay::SeqChunk ch;
      ch.tokens.assign(tp, tp + n_tokens[s]);
      ch.start_pos = start_pos[s];
      ch.block_table.assign(bp, bp + table_len[s]);
      ch.want_logits = want_logits ? want_logits[s] != 0 : true;
      b.seqs.push_back(ch);
      tp += n_tokens[s];
      bp += table_len[s];
    }
    std::vector<float> lg = h->be->forward(b);
    if (lg.size() > cap) throw std::invalid_argument("logits buffer too small");
    if (!lg.empty()) std::memcpy(logits, lg.data(), lg.size() * 4);
    return static_cast<int>(lg.size() / h->w.config.vocab);
  } catch (const std::exception& e) {
    g_error = e.what();
    return -1;
  }
}

// Greedy generation through the reference Engine (engine.cpp:173-318): max_new tokens
// after the prompt; tokens to out_tokens, the logits each token was chosen from to
// out_logits (max_new * vocab floats, may be NULL).
int ref_generate(void* hp, const int* prompt, int n, int max_new, int max_batch_tokens, int* out_tokens,
                 float* out_logits) {
  auto* h = static_cast<Handle*>(hp);
  try {
    relay::Engine engine(*h->be, {max_batch_tokens, 8, false, false});
    const int V = h->w.config.vocab;
    int seen = 0;
    engine.on_logits = [&](std::uint64_t, int idx, const float* lg) {
      if (out_logits && idx < max_new) std::memcpy(out_logits + static_cast<std::size_t>(idx) * V, lg, V * 4);
      ++seen;
    };
    relay::SamplingParams sp;
    sp.max_new_tokens = max_new;
    sp.ignore_eos = true;
    engine.add({1, std::vector<int>(prompt, prompt + n), sp});
    auto out = engine.run_all();
    const auto& toks = out[1];
    for (std::size_t i = 0; i < toks.size(); ++i) out_tokens[i] = toks[i];
    return static_cast<int>(toks.size());
  } catch (const std::exception& e) {
    g_error = e.what();
    return -1;
  }
}

// Backend::write_kv_block of the reference CPU backend (fp32 blocks, cpu_backend.cpp:79-83).
int ref_write_kv_block(void* hp, int layer, int block, const float* k, const float* v) {
  try {
    static_cast<Handle*>(hp)->be->write_kv_block(layer, block, k, v);
    return 0;
  } catch (const std::exception& e) {
    g_error = e.what();
    return -1;
  }
}

void ref_f32_to_f16(const float* in, std::uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = relay::f32_to_f16(in[i]);
}

int ref_rope_inv_freq(void* hp, float* out) {
  auto v = static_cast<Handle*>(hp)->w.config.rope_inv_freq();
  std::memcpy(out, v.data(), v.size() * 4);
  return static_cast<int>(v.size());
}

// A fused weight of the loaded model by relay's name, copied out (HostWeights layout).
long ref_weight(void* hp, const char* name, float* out, size_t cap) {
  auto& w = static_cast<Handle*>(hp)->w;
  std::string n = name;
  const std::vector<float>* v = nullptr;
  if (n == "embed") v = &w.embed;
  else if (n == "final_norm") v = &w.final_norm;
  else if (n == "lm_head") v = &w.lm_head;
  else if (n.rfind("layers.", 0) == 0) {
    std::size_t dot = n.find('.', 7);
    int i = std::stoi(n.substr(7, dot - 7));
    std::string f = n.substr(dot + 1);
    auto& L = w.layers.at(i);
    if (f == "attn_norm") v = &L.attn_norm;
    else if (f == "wqkv") v = &L.wqkv;
    else if (f == "bqkv") v = &L.bqkv;
    else if (f == "wo") v = &L.wo;
    else if (f == "mlp_norm") v = &L.mlp_norm;
    else if (f == "w_gate_up") v = &L.w_gate_up;
    else if (f == "w_down") v = &L.w_down;
  }
  if (!v) return -1;
  if (out && v->size() <= cap) std::memcpy(out, v->data(), v->size() * 4);
  return static_cast<long>(v->size());
}

}  // extern "C"
