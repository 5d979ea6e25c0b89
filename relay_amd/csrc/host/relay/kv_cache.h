// The paged KV cache's layout: relay's KVLayout (engine/include/relay/kv_cache.h:20-37).
// Per layer, K and V each [block][kv_head][slot][head_dim]; position p of a sequence is
// in block table[p / block_size], slot p % block_size.
#pragma once

#include <cstdint>

namespace relay {

struct KVLayout {
  int layers = 0;
  int kv_heads = 0;
  int head_dim = 0;
  int block_size = 16;
  int num_blocks = 0;

  std::int64_t block_elems() const { return static_cast<std::int64_t>(kv_heads) * block_size * head_dim; }
  std::int64_t layer_elems() const { return block_elems() * num_blocks; }
  std::int64_t offset(int block, int kv_head, int slot) const {
    return (static_cast<std::int64_t>(block) * kv_heads + kv_head) * block_size * head_dim +
           static_cast<std::int64_t>(slot) * head_dim;
  }
  int blocks_for(int tokens) const { return (tokens + block_size - 1) / block_size; }
};

}  // namespace relay
