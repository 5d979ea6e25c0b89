// relay's backend boundary (engine/include/relay/backend.h:20-98), restated for this
// build: SeqChunk / ForwardBatch / LayerObserver / Backend with the same members and
// contracts, plus the HIP backend's factory and options. Backend code here compiles
// unchanged against relay's own header once make_hip_backend and HipOptions are added
// there (the integration notes show the lines).
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "relay/config.h"
#include "relay/kv_cache.h"
#include "relay/weights.h"

namespace relay {

struct SeqChunk {
  std::vector<int> tokens;       // the new tokens
  int start_pos = 0;             // position of tokens[0]; earlier positions are in the cache
  std::vector<int> block_table;  // covers positions [0, start_pos + tokens.size())
  bool want_logits = true;       // logits for the chunk's last token (or all, see ForwardBatch)
};

struct ForwardBatch {
  std::vector<SeqChunk> seqs;
  bool all_logits = false;  // logits for every token instead of each chunk's last
};

class LayerObserver {
 public:
  virtual ~LayerObserver() = default;
  virtual void kv_written(int layer) = 0;
};

class Backend {
 public:
  virtual ~Backend() = default;
  virtual const ModelConfig& config() const = 0;
  virtual const KVLayout& kv_layout() const = 0;
  virtual std::string name() const = 0;
  // Writes each token's K and V into the cache; returns fp32 logits [rows, vocab].
  virtual std::vector<float> forward(const ForwardBatch& batch, LayerObserver* observer = nullptr) = 0;
  virtual std::size_t kv_block_bytes() const = 0;
  virtual void read_kv_block(int layer, int block, void* k_out, void* v_out) = 0;
  virtual void write_kv_block(int layer, int block, const void* k_in, const void* v_in) = 0;
  // out = all K blocks then all V blocks, in the order given.
  virtual void read_kv_layer(int layer, const std::vector<int>& blocks, void* out);
  virtual void write_kv_layer(int layer, const std::vector<int>& blocks, const void* in);
  virtual void* kv_host_ptr(int layer, int block, bool value) { return nullptr; }
  virtual void wait_kv_written(int layer) {}
  virtual void update_weight(const std::string& name, const float* src, std::size_t n);
};

// Options of the HIP backend (the counterpart of CudaOptions, backend.h:85-94).
struct HipOptions {
  // The reference attention kernel everywhere instead of the split decode and flash
  // prefill kernels (tests compare the two; also the path for head sizes the fast
  // kernels do not cover).
  bool reference_attention = false;
  // Weight-only int8 for the transformer layers' matrices (one scale per output row).
  bool int8_weights = false;
  // From the environment: RELAY_HIP_ATTENTION=ref, RELAY_HIP_INT8=1.
  static HipOptions from_env();
};

std::unique_ptr<Backend> make_hip_backend(const HostWeights& weights, int num_blocks, int block_size, int device,
                                          int max_batch_tokens, int max_context,
                                          HipOptions options = HipOptions::from_env());

}  // namespace relay
