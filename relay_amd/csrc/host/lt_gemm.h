// The dense projections above the skinny product's token range, through hipBLASLt with the
// kernel picked by timing: y[T, N] (fp32) = x[T, K] (fp16) W[N, K]^T (fp16) + beta y.
//
// relay calls cublasGemmEx with the library's default choice (cuda_backend.cu:726-730). On
// this stack the default choice is not the fastest kernel the libraries have for some
// shapes (Llama-3-8B down projection at 560 tokens, 4096 x 14336, in a forward pass: 114 us
// with rocBLAS' choice, 100 us with the fastest of hipBLASLt's heuristic candidates), so the
// first call of each (token-count bucket, N, K) times up to kCandidates candidates, each
// with the weights evicted from the caches first, and keeps the fastest.
#pragma once

#include <hip/hip_runtime_api.h>
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <memory>
#include <tuple>

#include "host_common.h"

namespace relay_hip_host {

class LtGemm {
 public:
  explicit LtGemm(hipStream_t stream);
  ~LtGemm();
  LtGemm(const LtGemm&) = delete;
  LtGemm& operator=(const LtGemm&) = delete;

  // Runs the product; false if hipBLASLt has no algorithm for the shape (the caller falls
  // back). The first call of a (bucket, N, K) times the candidates into a scratch output,
  // so y is written once whatever beta is.
  bool run(const void* W, const void* x, float* y, int T, int K, int N, float beta);

  // 64 rather than 16 heuristic candidates: TinyLlama's 32 x 2048 decode step 1.70 -> 1.66 ms
  // (its 32-token products), the 2048-token prefill and the Llama-3 mixed step level.
  static constexpr int kCandidates = 64;
  static constexpr std::size_t kWorkspaceBytes = std::size_t(128) << 20;
  // Written before each timed candidate call: more than the 256 MB Infinity Cache.
  static constexpr std::size_t kFlushBytes = std::size_t(320) << 20;

 private:
  // Descriptors of one exact shape, and the algorithm it runs (valid = usable).
  struct Shape {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    bool valid = false;
  };
  Shape& shape(const void* W, const void* x, int T, int K, int N);
  bool tune(Shape& s, const void* W, const void* x, int T, int K, int N, hipblasLtMatmulAlgo_t& best);
  bool supported(Shape& s, hipblasLtMatmulAlgo_t& algo);

  hipStream_t stream_;
  hipblasLtHandle_t handle_ = nullptr;
  DeviceArray<unsigned char> workspace_;
  DeviceArray<float> scratch_;
  hipEvent_t ev_[2] = {nullptr, nullptr};
  std::map<std::tuple<int, int, int>, std::unique_ptr<Shape>> shapes_;  // exact (T, N, K)
  std::map<std::tuple<int, int, int>, hipblasLtMatmulAlgo_t> tuned_;    // (bucket of T, N, K)
};

}  // namespace relay_hip_host
