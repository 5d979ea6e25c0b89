// The default implementations relay's Backend declares (engine/src/backend.cpp:10-24):
// layer-wide KV I/O as a loop over blocks, and update_weight refusing. Only for this
// build's own boundary header; with relay's headers, relay's backend.cpp provides them.
#include <stdexcept>

#include "relay/backend.h"

namespace relay {

void Backend::update_weight(const std::string& name, const float* src, std::size_t n) {
  throw std::logic_error(this->name() + " backend: update_weight is not supported; write the host weights");
}

void Backend::read_kv_layer(int layer, const std::vector<int>& blocks, void* out) {
  const std::size_t bb = kv_block_bytes(), n = blocks.size();
  auto* k = static_cast<unsigned char*>(out);
  for (std::size_t i = 0; i < n; ++i) read_kv_block(layer, blocks[i], k + i * bb, k + (n + i) * bb);
}

void Backend::write_kv_layer(int layer, const std::vector<int>& blocks, const void* in) {
  const std::size_t bb = kv_block_bytes(), n = blocks.size();
  const auto* k = static_cast<const unsigned char*>(in);
  for (std::size_t i = 0; i < n; ++i) write_kv_block(layer, blocks[i], k + i * bb, k + (n + i) * bb);
}

}  // namespace relay
