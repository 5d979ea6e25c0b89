// Model hyperparameters: the fields of relay's ModelConfig (engine/include/relay/config.h)
// that a backend reads. Same names and meanings, so backend code written against this
// header compiles unchanged against relay's own.
#pragma once

#include <string>
#include <vector>

namespace relay {

struct RopeScaling {
  std::string type;  // "" (none) or "llama3"
  double factor = 1;
  double low_freq_factor = 1;
  double high_freq_factor = 4;
  double original_max_position = 8192;
};

struct ModelConfig {
  std::string model_type;
  int hidden = 0;
  int intermediate = 0;
  int layers = 0;
  int heads = 0;
  int kv_heads = 0;
  int head_dim = 0;
  int vocab = 0;
  int max_position = 0;
  double rms_eps = 1e-5;
  double rope_theta = 10000;
  RopeScaling rope_scaling;
  bool tie_embeddings = false;
  bool qkv_bias = false;
  std::vector<int> eos_ids;

  int q_dim() const { return heads * head_dim; }
  int kv_dim() const { return kv_heads * head_dim; }

  // head_dim / 2 inverse rotary frequencies, Llama 3 scaling applied when configured
  // (relay's formula, config.cpp:79-109).
  std::vector<float> rope_inv_freq() const;
};

}  // namespace relay
