// ModelConfig::rope_inv_freq for this build's boundary headers: the inverse rotary
// frequencies 1 / theta^(2i / head_dim) in float32 (how transformers computes them from
// an integer range), with Llama 3's piecewise band scaling when configured. The formula
// must equal relay's (config.cpp:79-109) bit for bit, since both CPU and GPU backends
// rotate with it; tests compare the two.
#include <cmath>

#include "relay/config.h"

namespace relay {

std::vector<float> ModelConfig::rope_inv_freq() const {
  const int half = head_dim / 2;
  std::vector<float> inv(half);
  for (int i = 0; i < half; ++i)
    inv[i] = 1.0f / std::pow(static_cast<float>(rope_theta), static_cast<float>(2 * i) / static_cast<float>(head_dim));
  if (rope_scaling.type != "llama3") return inv;
  const RopeScaling& rs = rope_scaling;
  // Wavelengths above original_max / low_freq_factor are slowed by `factor`; those
  // below original_max / high_freq_factor are kept; in between, a linear blend in
  // (original_max / wavelength).
  const double long_wave = rs.original_max_position / rs.low_freq_factor;
  const double short_wave = rs.original_max_position / rs.high_freq_factor;
  const float two_pi = 2.0f * static_cast<float>(M_PI);
  const float factor = static_cast<float>(rs.factor);
  for (int i = 0; i < half; ++i) {
    const float f = inv[i];
    const float wavelen = two_pi / f;
    if (wavelen > long_wave) {
      inv[i] = f / factor;
    } else if (wavelen < short_wave) {
      inv[i] = f;
    } else {
      const float blend = static_cast<float>((rs.original_max_position / wavelen - rs.low_freq_factor) /
                                             (rs.high_freq_factor - rs.low_freq_factor));
      inv[i] = (1 - blend) * f / factor + blend * f;
    }
  }
  return inv;
}

}  // namespace relay
