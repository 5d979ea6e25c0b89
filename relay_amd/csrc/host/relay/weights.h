// Host fp32 weights in relay's fused layout (engine/include/relay/weights.h:13-31):
// q/k/v fused into wqkv, gate/up into w_gate_up; lm_head empty when tied to embed.
#pragma once

#include <vector>

#include "relay/config.h"

namespace relay {

struct LayerWeights {
  std::vector<float> attn_norm;  // [hidden]
  std::vector<float> wqkv;       // [q_dim + 2 * kv_dim, hidden]
  std::vector<float> bqkv;       // [q_dim + 2 * kv_dim] or empty
  std::vector<float> wo;         // [hidden, q_dim]
  std::vector<float> mlp_norm;   // [hidden]
  std::vector<float> w_gate_up;  // [2 * intermediate, hidden]: gate rows, then up rows
  std::vector<float> w_down;     // [hidden, intermediate]
};

struct HostWeights {
  ModelConfig config;
  std::vector<float> embed;       // [vocab, hidden]
  std::vector<LayerWeights> layers;
  std::vector<float> final_norm;  // [hidden]
  std::vector<float> lm_head;     // [vocab, hidden]; empty when tied to embed

  const std::vector<float>& lm_head_or_embed() const { return lm_head.empty() ? embed : lm_head; }
};

}  // namespace relay
