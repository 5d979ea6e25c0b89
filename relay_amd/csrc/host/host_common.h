// Host-side helpers of the HIP backend: owning device and pinned-host buffers and the
// error-check macros (runtime failures become std::runtime_error, as relay's CUDA
// backend does with its CUDA_CHECK).
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <stdexcept>
#include <string>

#include "relay_hip.h"

#define HIP_CHECK(x)                                                                          \
  do {                                                                                        \
    hipError_t _e = (x);                                                                      \
    if (_e != hipSuccess) throw std::runtime_error(std::string("HIP: ") + hipGetErrorString(_e) + " at " #x); \
  } while (0)

#define RH_CHECK(x)                                                                           \
  do {                                                                                        \
    if ((x) != 0) throw std::runtime_error(std::string("relay_hip: ") + rh_last_error() + " at " #x); \
  } while (0)

namespace relay_hip_host {

// An owning device allocation of n elements.
template <class T>
struct DeviceArray {
  T* p = nullptr;
  std::size_t n = 0;
  DeviceArray() = default;
  explicit DeviceArray(std::size_t count) : n(count) {
    if (count) HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&p), count * sizeof(T)));
  }
  ~DeviceArray() { reset(); }
  DeviceArray(const DeviceArray&) = delete;
  DeviceArray& operator=(const DeviceArray&) = delete;
  DeviceArray(DeviceArray&& o) noexcept : p(o.p), n(o.n) {
    o.p = nullptr;
    o.n = 0;
  }
  DeviceArray& operator=(DeviceArray&& o) noexcept {
    if (this != &o) {
      reset();
      p = o.p;
      n = o.n;
      o.p = nullptr;
      o.n = 0;
    }
    return *this;
  }
  void reset() {
    if (p) (void)hipFree(p);
    p = nullptr;
    n = 0;
  }
};

// Page-locked host memory that only grows (copies from it run asynchronously).
struct PinnedBuffer {
  void* p = nullptr;
  std::size_t bytes = 0;
  PinnedBuffer() = default;
  PinnedBuffer(const PinnedBuffer&) = delete;
  PinnedBuffer& operator=(const PinnedBuffer&) = delete;
  ~PinnedBuffer() {
    if (p) (void)hipHostFree(p);
  }
  void reserve(std::size_t want) {
    if (want <= bytes) return;
    if (p) HIP_CHECK(hipHostFree(p));
    p = nullptr;
    const std::size_t grow = want + want / 2;
    HIP_CHECK(hipHostMalloc(&p, grow, hipHostMallocDefault));
    bytes = grow;
  }
};

}  // namespace relay_hip_host
