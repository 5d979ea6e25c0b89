// relay's Backend on one MI355X: fp16 (or weight-only int8) weights and KV cache in HBM,
// fp32 residual stream, the gfx950 kernels of include/relay_hip.h for attention and the
// int8 GEMV, rocBLAS for the dense fp16 GEMMs.
//
// The host orchestration mirrors CudaBackend (engine/src/cuda_backend.cu:311-759) in
// contract, not in code:
//  - a forward pass flattens the batch (cuda_backend.cu:508-527), routes single-token
//    chunks to the split decode kernel and longer chunks to flash prefill
//    (cuda_backend.cu:528-545), runs the layers, and returns fp32 logits;
//  - the per-step metadata goes to the device in ONE copy from a pinned buffer (the
//    reference issues seven); the prefill work (rh_prefill_plan) pairs light and heavy
//    causal row blocks and comes heaviest first, so the imbalance does not leave CUs
//    idle at the end of the kernel;
//  - one event per layer after its KV write backs wait_kv_written, and KV block traffic
//    runs on a second stream under its own mutex (cuda_backend.cu:611-664).
// Errors are C++ exceptions as in the reference: std::invalid_argument for bad batches,
// std::out_of_range for token ids, std::runtime_error("HIP: ...") for runtime failures.
#include <hip/hip_runtime_api.h>
#include <rocblas/rocblas.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <functional>
#include <limits>
#include <memory>
#include <mutex>
#include <numeric>
#include <stdexcept>
#include <string>
#include <system_error>
#include <thread>

#include "relay/backend.h"
#include "relay_hip.h"
#include "host_common.h"
#include "lt_gemm.h"

namespace relay {

HipOptions HipOptions::from_env() {
  HipOptions o;
  if (const char* a = std::getenv("RELAY_HIP_ATTENTION")) o.reference_attention = std::string(a) == "ref";
  if (const char* q = std::getenv("RELAY_HIP_INT8")) o.int8_weights = std::string(q) == "1";
  return o;
}

namespace {

using relay_hip_host::DeviceArray;
using relay_hip_host::PinnedBuffer;
using relay_hip_host::LtGemm;


#define ROCBLAS_CHECK(x)                                                                          \
  do {                                                                                            \
    rocblas_status _s = (x);                                                                      \
    if (_s != rocblas_status_success)                                                             \
      throw std::runtime_error(std::string("rocBLAS: ") + rocblas_status_to_string(_s) + " at " #x); \
  } while (0)

// A weight matrix [N, K]: fp16, or int8 with one fp32 scale per row (int8 rows ldw bytes
// apart, rh_gemv_int8_row_stride).
struct DeviceMatrix {
  int N = 0, K = 0;
  std::int64_t ldw = 0;
  DeviceArray<std::uint16_t> f16;
  DeviceArray<std::int8_t> i8;
  DeviceArray<float> scale;
};

struct DeviceLayer {
  DeviceArray<float> attn_norm, mlp_norm, bqkv;
  DeviceMatrix wqkv, wo, w_gate_up, w_down;
};

// Where construction takes its weights from: host fp32 arrays (relay's HostWeights
// layout) or a seeded draw on the device.
struct WeightSource {
  const rh_host_weights* host = nullptr;
  bool synthetic = false;
  std::uint64_t seed = 0;
  float std = 0.02f;
};

class HipBackend final : public Backend {
 public:
  HipBackend(const ModelConfig& c, const WeightSource& src, int num_blocks, int block_size, int device,
             int max_tokens, int max_context, HipOptions options)
      : c_(c), opt_(options), max_tokens_(max_tokens), max_context_(max_context), device_(device) {
    if (num_blocks <= 0 || block_size <= 0) throw std::invalid_argument("num_blocks and block_size must be positive");
    if (max_tokens <= 0) throw std::invalid_argument("max_batch_tokens must be positive");
    if (c.heads <= 0 || c.kv_heads <= 0 || c.heads % c.kv_heads) throw std::invalid_argument("bad head counts");
    HIP_CHECK(hipSetDevice(device));
    HIP_CHECK(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
    HIP_CHECK(hipStreamCreateWithFlags(&copy_stream_, hipStreamNonBlocking));
    HIP_CHECK(hipEventCreate(&fwd_begin_));
    HIP_CHECK(hipEventCreate(&fwd_end_));
    ROCBLAS_CHECK(rocblas_create_handle(&blas_));
    ROCBLAS_CHECK(rocblas_set_stream(blas_, stream_));
    // RELAY_HIP_GEMM=rocblas keeps every library product on rocBLAS' own choice.
    const char* g = std::getenv("RELAY_HIP_GEMM");
    if (!(g && std::string(g) == "rocblas")) lt_ = std::make_unique<LtGemm>(stream_);
    layer_done_.resize(c_.layers);
    for (auto& e : layer_done_) HIP_CHECK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    layout_ = {c_.layers, c_.kv_heads, c_.head_dim, block_size, num_blocks};
    if (kv_block_bytes() % 16 != 0) throw std::invalid_argument("a KV block must be a multiple of 16 bytes");
    const int D = c_.head_dim;
    fast_attention_ = !opt_.reference_attention && (D == 16 || D == 32 || D == 64 || D == 128);
    if (!fast_attention_ && D > 256) throw std::invalid_argument("head_dim above 256 is not supported");

    load_weights(src);

    kc_ = DeviceArray<std::uint16_t>(static_cast<std::size_t>(layout_.layer_elems()) * c_.layers);
    vc_ = DeviceArray<std::uint16_t>(kc_.n);
    HIP_CHECK(hipMemset(kc_.p, 0, kc_.n * 2));
    HIP_CHECK(hipMemset(vc_.p, 0, vc_.n * 2));

    const std::size_t T = max_tokens_;
    const int H = c_.hidden, QKV = c_.q_dim() + 2 * c_.kv_dim(), I = c_.intermediate;
    x_ = DeviceArray<float>(T * H);
    xn_ = DeviceArray<std::uint16_t>(T * std::max(H, I));
    qkv_ = DeviceArray<float>(T * QKV);
    qh_ = DeviceArray<std::uint16_t>(T * c_.q_dim());
    attn_ = DeviceArray<std::uint16_t>(T * c_.q_dim());
    gu_ = DeviceArray<float>(T * 2 * I);
    act_ = DeviceArray<std::uint16_t>(T * I);
    logits_ = DeviceArray<float>(T * c_.vocab);
    HIP_CHECK(hipStreamSynchronize(stream_));
  }

  ~HipBackend() override {
    (void)hipSetDevice(device_);
    if (stream_) (void)hipStreamSynchronize(stream_);
    if (copy_stream_) (void)hipStreamSynchronize(copy_stream_);
    if (blas_) rocblas_destroy_handle(blas_);
    for (auto e : layer_done_) (void)hipEventDestroy(e);
    for (auto e : kv_events_) (void)hipEventDestroy(e);
    for (auto e : logit_events_) (void)hipEventDestroy(e);
    if (fwd_begin_) (void)hipEventDestroy(fwd_begin_);
    if (fwd_end_) (void)hipEventDestroy(fwd_end_);
    if (stream_) (void)hipStreamDestroy(stream_);
    if (copy_stream_) (void)hipStreamDestroy(copy_stream_);
  }

  const ModelConfig& config() const override { return c_; }
  const KVLayout& kv_layout() const override { return layout_; }
  std::string name() const override { return "hip"; }
  std::size_t kv_block_bytes() const override { return static_cast<std::size_t>(layout_.block_elems()) * 2; }

  double last_forward_ms() const { return last_ms_; }

  void read_kv_block(int layer, int block, void* k_out, void* v_out) override {
    HIP_CHECK(hipSetDevice(device_));
    kv_io(layer, {block}, k_out, v_out, nullptr, nullptr);
  }
  void write_kv_block(int layer, int block, const void* k_in, const void* v_in) override {
    HIP_CHECK(hipSetDevice(device_));
    kv_io(layer, {block}, nullptr, nullptr, k_in, v_in);
  }
  void read_kv_layer(int layer, const std::vector<int>& blocks, void* out) override {
    HIP_CHECK(hipSetDevice(device_));
    auto* k = static_cast<unsigned char*>(out);
    kv_io(layer, blocks, k, k + blocks.size() * kv_block_bytes(), nullptr, nullptr);
  }
  void write_kv_layer(int layer, const std::vector<int>& blocks, const void* in) override {
    HIP_CHECK(hipSetDevice(device_));
    const auto* k = static_cast<const unsigned char*>(in);
    kv_io(layer, blocks, nullptr, nullptr, k, k + blocks.size() * kv_block_bytes());
  }
  void wait_kv_written(int layer) override { HIP_CHECK(hipEventSynchronize(layer_done_.at(layer))); }

  void update_weight(const std::string& name, const float* src, std::size_t n) override;

  void fill_kv_random(std::uint64_t seed, float std) {
    HIP_CHECK(hipSetDevice(device_));
    RH_CHECK(rh_fill_normal_f16(kc_.p, kc_.n, seed, 1000001, 0.0f, std, stream_));
    RH_CHECK(rh_fill_normal_f16(vc_.p, vc_.n, seed, 1000002, 0.0f, std, stream_));
    HIP_CHECK(hipStreamSynchronize(stream_));
  }

  std::vector<float> forward(const ForwardBatch& batch, LayerObserver* observer) override;
  // forward() with the logits rows written straight into dst (cap floats; the C ABI's
  // caller buffer), no intermediate vector. Returns the number of rows.
  int forward_into(const ForwardBatch& batch, float* dst, std::size_t cap);

 private:
  // Everything of a forward pass up to the logits on the device; returns their count
  // (rows x vocab), throws before launching anything if that exceeds cap.
  std::size_t enqueue_forward(const ForwardBatch& batch, LayerObserver* observer, std::size_t cap);
  // Waits for the pass and copies its n logits to dst: device -> pinned in pieces, each piece
  // copied on to dst as soon as it lands, under the DMA of the next.
  void finish_forward(float* dst, std::size_t n);
  static constexpr int kLogitChunks = 16;
  // Each D2H piece costs ~10 us of its own beyond its bytes: TinyLlama's 4 MB of logits for
  // 32 rows took 0.43 ms from the forward's end to the caller's buffer in 16 pieces of 256
  // KB, 0.29 ms in 4 of 1 MB (one piece then 4 threads: 0.33 ms); 25 MB in 16 pieces level.
  static constexpr std::size_t kLogitMinPiece = std::size_t(1) << 20;
  static constexpr int kLogitThreads = 4;
  static constexpr std::size_t kLogitThreadBytes = std::size_t(2) << 20;
  std::vector<hipEvent_t> logit_events_;
  bool pending_ = false;  // a pass was enqueued and not yet finished
  void load_weights(const WeightSource& src);
  DeviceMatrix make_matrix(const float* host, int N, int K, const WeightSource& src, std::uint64_t stream_id);
  DeviceArray<std::uint16_t> make_f16(const float* host, std::size_t n, const WeightSource& src,
                                      std::uint64_t stream_id);
  DeviceArray<float> make_f32(const float* host, std::size_t n, float fill);
  void upload_f32_rows(const float* host, int N, int K, const std::function<void(const float*, int, int)>& apply);
  void gemm(const DeviceMatrix& W, const std::uint16_t* x, float* y, int T, float beta);
  // int8_ok: the caller has an int8 variant of the fused product (the qkv projection).
  bool fused(const DeviceMatrix& W, int T, bool int8_ok = false) const;
  float* w8_split_ws(int ks, int T, int N);
  int w8_partials(const DeviceMatrix& W, const std::uint16_t* x, int T);
  void gemm_f16(const std::uint16_t* W, const std::uint16_t* x, float* y, int T, int K, int N, float beta);
  // Whether gemm_f16 runs the skinny product (else the library GEMM) for this shape.
  static bool skinny(int K, int N, int T);
  void kv_io(int layer, const std::vector<int>& blocks, void* k_out, void* v_out, const void* k_in, const void* v_in);
  // Pieces of one KV transfer: writes in up to 16, reads in up to 8 (each DMA piece costs
  // ~10 us beyond its bytes, and a read's host copies are split over the threads; Llama-3
  // layer reads of 33.6 MB: 34.1 GB/s at 16 pieces, 36.9-38.8 at 8, 38.5-39.1 at 4, 28-31 at 2;
  // writes 35.5 at 16, 34-36 at 8, 30.5 at 4).
  static constexpr int kKvChunks = 16, kKvReadChunks = 8;
  static constexpr int kKvThreads = 4;                          // host threads copying them (8: no faster)
  static constexpr std::size_t kKvMinPiece = std::size_t(1) << 20;
  std::vector<hipEvent_t> kv_events_;                           // one per piece in flight

  ModelConfig c_;
  HipOptions opt_;
  bool fast_attention_ = false;
  KVLayout layout_;
  int max_tokens_, max_context_, device_;
  hipStream_t stream_ = nullptr, copy_stream_ = nullptr;
  rocblas_handle blas_ = nullptr;
  std::unique_ptr<LtGemm> lt_;  // timed-choice hipBLASLt products (rocBLAS if it has none)
  std::vector<hipEvent_t> layer_done_;
  hipEvent_t fwd_begin_ = nullptr, fwd_end_ = nullptr;
  double last_ms_ = 0;

  DeviceArray<std::uint16_t> embed_, lm_head_;
  DeviceArray<float> final_norm_, inv_freq_;
  std::vector<DeviceLayer> layers_;
  DeviceArray<std::uint16_t> kc_, vc_;
  DeviceArray<float> x_, qkv_, gu_, logits_;
  DeviceArray<std::uint16_t> xn_, qh_, attn_, act_;
  DeviceArray<std::uint16_t> dequant_;  // int8 weights widened (K % 64 != 0, above the GEMV's limit)
  std::size_t dequant_elems_ = 0;
  DeviceArray<float> stage_;            // fp32 staging for uploads and update_weight

  // Per-step metadata: one pinned host buffer, one device buffer, one copy.
  PinnedBuffer meta_host_;
  DeviceArray<int> meta_dev_;
  PinnedBuffer logits_host_;
  DeviceArray<float> part_o_, part_ml_;
  DeviceArray<int> counters_;
  DeviceArray<float> split_ws_;      // K-range partials of the split skinny product
  DeviceArray<int> split_counters_;  // its per-tile arrival counters (zero between calls)

  std::mutex copy_mu_;
  DeviceArray<unsigned char> kv_stage_dev_;
  DeviceArray<int> kv_ids_dev_;
  PinnedBuffer kv_stage_host_;
};

void HipBackend::upload_f32_rows(const float* host, int N, int K,
                                 const std::function<void(const float*, int, int)>& apply) {
  // Row-aligned chunks of at most 16M floats through the fp32 staging buffer.
  const std::size_t rows_per = std::max<std::size_t>(1, (std::size_t(16) << 20) / static_cast<std::size_t>(K));
  const std::size_t need = std::min<std::size_t>(N, rows_per) * K;
  if (stage_.n < need) stage_ = DeviceArray<float>(need);
  for (int r0 = 0; r0 < N; r0 += static_cast<int>(rows_per)) {
    const int rows = std::min<int>(static_cast<int>(rows_per), N - r0);
    HIP_CHECK(hipMemcpyAsync(stage_.p, host + static_cast<std::size_t>(r0) * K, static_cast<std::size_t>(rows) * K * 4,
                             hipMemcpyHostToDevice, stream_));
    apply(stage_.p, r0, rows);
  }
}

DeviceArray<std::uint16_t> HipBackend::make_f16(const float* host, std::size_t n, const WeightSource& src,
                                                std::uint64_t stream_id) {
  DeviceArray<std::uint16_t> d(n);
  if (src.synthetic) {
    RH_CHECK(rh_fill_normal_f16(d.p, n, src.seed, stream_id, 0.0f, src.std, stream_));
    return d;
  }
  // Viewed as rows of 4096 (plus a tail row) for the chunked upload.
  const int K = 4096;
  const int full = static_cast<int>(n / K);
  if (full)
    upload_f32_rows(host, full, K, [&](const float* chunk, int r0, int rows) {
      RH_CHECK(rh_f32_to_f16(chunk, d.p + static_cast<std::size_t>(r0) * K, static_cast<std::size_t>(rows) * K, stream_));
    });
  const std::size_t tail = n - static_cast<std::size_t>(full) * K;
  if (tail)
    upload_f32_rows(host + static_cast<std::size_t>(full) * K, 1, static_cast<int>(tail), [&](const float* chunk, int, int) {
      RH_CHECK(rh_f32_to_f16(chunk, d.p + static_cast<std::size_t>(full) * K, tail, stream_));
    });
  return d;
}

DeviceArray<float> HipBackend::make_f32(const float* host, std::size_t n, float fill) {
  DeviceArray<float> d(n);
  if (!n) return d;
  if (host) {
    HIP_CHECK(hipMemcpyAsync(d.p, host, n * 4, hipMemcpyHostToDevice, stream_));
  } else {
    std::vector<float> v(n, fill);
    HIP_CHECK(hipMemcpy(d.p, v.data(), n * 4, hipMemcpyHostToDevice));
  }
  HIP_CHECK(hipStreamSynchronize(stream_));
  return d;
}

DeviceMatrix HipBackend::make_matrix(const float* host, int N, int K, const WeightSource& src,
                                     std::uint64_t stream_id) {
  DeviceMatrix m;
  m.N = N;
  m.K = K;
  const std::size_t n = static_cast<std::size_t>(N) * K;
  if (!opt_.int8_weights) {
    m.f16 = make_f16(host, n, src, stream_id);
    return m;
  }
  m.ldw = rh_gemv_int8_row_stride(K);
  m.i8 = DeviceArray<std::int8_t>(static_cast<std::size_t>(N) * static_cast<std::size_t>(m.ldw));
  m.scale = DeviceArray<float>(N);
  if (src.synthetic) {
    // fp32 rows drawn on the device, then the same quantizer as the host-weight path.
    const std::size_t rows_per = std::max<std::size_t>(1, (std::size_t(16) << 20) / static_cast<std::size_t>(K));
    if (stage_.n < std::min<std::size_t>(N, rows_per) * K) stage_ = DeviceArray<float>(std::min<std::size_t>(N, rows_per) * K);
    for (int r0 = 0; r0 < N; r0 += static_cast<int>(rows_per)) {
      const int rows = std::min<int>(static_cast<int>(rows_per), N - r0);
      RH_CHECK(rh_fill_normal_f32(stage_.p, static_cast<std::size_t>(rows) * K, src.seed, stream_id * 65536 + r0, 0.0f,
                                  src.std, stream_));
      RH_CHECK(rh_quantize_int8(stage_.p, rows, K, m.i8.p + static_cast<std::size_t>(r0) * m.ldw, m.ldw,
                                m.scale.p + r0, stream_));
    }
  } else {
    upload_f32_rows(host, N, K, [&](const float* chunk, int r0, int rows) {
      RH_CHECK(rh_quantize_int8(chunk, rows, K, m.i8.p + static_cast<std::size_t>(r0) * m.ldw, m.ldw,
                                m.scale.p + r0, stream_));
    });
  }
  if (K % 64) dequant_elems_ = std::max(dequant_elems_, n);  // the int8 GEMM needs K % 64 == 0
  return m;
}

void HipBackend::load_weights(const WeightSource& src) {
  const int H = c_.hidden, Q = c_.q_dim(), KV = c_.kv_dim(), I = c_.intermediate, V = c_.vocab;
  const int QKV = Q + 2 * KV;
  const rh_host_weights* hw = src.host;
  embed_ = make_f16(hw ? hw->embed : nullptr, static_cast<std::size_t>(V) * H, src, 1);
  if (!c_.tie_embeddings) {
    if (hw && !hw->lm_head) throw std::invalid_argument("lm_head is missing and the embeddings are not tied");
    lm_head_ = make_f16(hw ? hw->lm_head : nullptr, static_cast<std::size_t>(V) * H, src, 2);
  }
  final_norm_ = make_f32(hw ? hw->final_norm : nullptr, H, 1.0f);
  inv_freq_ = make_f32(c_.rope_inv_freq().data(), c_.head_dim / 2, 0.0f);
  for (int l = 0; l < c_.layers; ++l) {
    DeviceLayer d;
    const std::uint64_t sid = 100 + 16 * static_cast<std::uint64_t>(l);
    d.attn_norm = make_f32(hw ? hw->attn_norm[l] : nullptr, H, 1.0f);
    d.mlp_norm = make_f32(hw ? hw->mlp_norm[l] : nullptr, H, 1.0f);
    if (c_.qkv_bias) d.bqkv = make_f32(hw && hw->bqkv ? hw->bqkv[l] : nullptr, QKV, 0.0f);
    d.wqkv = make_matrix(hw ? hw->wqkv[l] : nullptr, QKV, H, src, sid + 1);
    d.wo = make_matrix(hw ? hw->wo[l] : nullptr, H, Q, src, sid + 2);
    d.w_gate_up = make_matrix(hw ? hw->w_gate_up[l] : nullptr, 2 * I, H, src, sid + 3);
    d.w_down = make_matrix(hw ? hw->w_down[l] : nullptr, H, I, src, sid + 4);
    layers_.push_back(std::move(d));
  }
  HIP_CHECK(hipStreamSynchronize(stream_));
  if (opt_.int8_weights && max_tokens_ > rh_gemv_int8_max_tokens() && dequant_elems_)
    dequant_ = DeviceArray<std::uint16_t>(dequant_elems_);
  stage_ = DeviceArray<float>();  // uploads are done; update_weight reallocates on demand
}

void HipBackend::gemm_f16(const std::uint16_t* W, const std::uint16_t* x, float* y, int T, int K, int N, float beta) {
  // Decode batch sizes up to 16 tokens: the skinny MFMA product; above, the library's timed
  // choice. Measured on whole decode steps (ms per step, skinny / library for every plain
  // product): TinyLlama 1.38 / 1.42 at 8 tokens, 1.51 / 1.45 at 16, 1.88 / 1.67 at 24,
  // 2.06 / 1.70 at 32; SmolLM2-135M 1.16 / 1.28 at 8, 1.60 / 1.70 at 16, 1.66 / 1.50 at 32;
  // one token: config 1's step 0.85 against 1.75 ms.
  if (skinny(K, N, T)) {
    const int ks = rh_gemv_f16_split_plan(T, K, N);
    if (ks > 1) {
      const std::size_t need = static_cast<std::size_t>(ks) * T * N;
      if (need > split_ws_.n) split_ws_ = DeviceArray<float>(need);
      const std::size_t tiles = (N + 15) / 16;
      if (tiles > split_counters_.n) {
        split_counters_ = DeviceArray<int>(tiles);
        HIP_CHECK(hipMemsetAsync(split_counters_.p, 0, tiles * sizeof(int), stream_));
      }
    }
    RH_CHECK(rh_gemv_f16_splitk(W, K, x, y, T, K, N, beta, ks, split_ws_.p, split_counters_.p, stream_));
    return;
  }
  // Library products of the fp16 weights: hipBLASLt with a timed choice. A dequantized int8
  // copy (just written, read from the caches) stays on rocBLAS: measured faster there
  // (Llama-3 int8 mixed step 26.0 vs 26.7 ms).
  if (lt_ && W != dequant_.p && lt_->run(W, x, y, T, K, N, beta)) return;
  // Row-major y[T, N] = x[T, K] W[N, K]^T is column-major y^T (N x T) = W^T-view (K x N)^T x^T.
  const float alpha = 1.0f;
  ROCBLAS_CHECK(rocblas_gemm_ex(blas_, rocblas_operation_transpose, rocblas_operation_none, N, T, K, &alpha, W,
                                rocblas_datatype_f16_r, K, x, rocblas_datatype_f16_r, K, &beta, y,
                                rocblas_datatype_f32_r, N, y, rocblas_datatype_f32_r, N, rocblas_datatype_f32_r,
                                rocblas_gemm_algo_standard, 0, 0));
}

bool HipBackend::skinny(int K, int N, int T) {
  // Up to 16 tokens always; 17-32 tokens on matrices under 4 Mi weights (the whole-line
  // kernel: SmolLM2-135M 32 x 640 decode step 1.50 -> 1.27 ms; TinyLlama's 2048 x 2048 o
  // projection at 32 tokens 1.569 -> 1.592 ms against the library's).
  return K % 16 == 0 && (T <= 16 || (T <= 32 && static_cast<std::int64_t>(N) * K < (std::int64_t{1} << 22)));
}

bool HipBackend::fused(const DeviceMatrix& W, int T, bool int8_ok) const {
  // Normalisation / activation folded into the skinny fp16 product, up to 16 tokens, when its
  // 16-row tiles fit one round of workgroups on the CUs: every workgroup repeats the
  // prologue, so on wider matrices the repeats cost more than the launch they save (TinyLlama
  // gate_up, 704 tiles, at T = 8: 27.7 us fused against 3.7 + 13.8 us for RMSNorm and the
  // library product). With int8 weights only the qkv projection takes its RMSNorm and
  // qkv_post (TinyLlama int8 decode steps, ms: b = 1 1.073 -> 1.042, b = 4 1.169 -> 1.141);
  // the SiLU prologue on the int8 down projection was no faster at b = 1, 8, 16 and slower at
  // b = 4 (1.169 -> 1.240), gate_up never has few enough tiles.
  return (!W.i8.p || int8_ok) && T <= 16 && W.K % 16 == 0 && (W.N + 15) / 16 <= 256 &&
         rh_gemv_f16_fused_fits(T, W.K);
}

// The K ranges of an int8 product that gemm() would split at this T, with its partials
// written to split_ws_ for a consumer that merges them (rh_w8_merge_silu /
// rh_w8_merge_rmsnorm, one launch fewer per product); 0 when gemm() does not split it.
int HipBackend::w8_partials(const DeviceMatrix& W, const std::uint16_t* x, int T) {
  if (!W.i8.p || T <= 16 || W.K % 64 || W.N % 4) return 0;
  int ks = 0;
  if (T <= 64) {
    // Narrow matrices (the o projection) too from 25 tokens, where the merge folds the
    // MLP RMSNorm launch in (TinyLlama int8 decode at 28 / 32 / 40 / 48 / 64 sequences
    // -0.4..-0.7 / -1.0 / -3.1 / -3.5 / -5.5%, Llama-3-8B int8 48 x 8192 12.49 -> 12.31 ms;
    // at 17-24 level or slower).
    if (W.N >= 8192 || W.K >= 5000 || T > 24) ks = rh_gemm_w8_split_plan(T, W.K, W.N);
  } else {
    ks = rh_gemm_w8_partials_plan(T, W.K, W.N);
  }
  if (ks < 2) return 0;
  RH_CHECK(rh_gemm_w8_partials(W.i8.p, W.ldw, x, T, W.K, W.N, ks, w8_split_ws(ks, T, W.N), stream_));
  return ks;
}

// The K-range workspace of a split int8 product (grown on demand).
float* HipBackend::w8_split_ws(int ks, int T, int N) {
  if (ks <= 1) return nullptr;
  const std::size_t need = static_cast<std::size_t>(ks) * T * N;
  if (need > split_ws_.n) split_ws_ = DeviceArray<float>(need);
  return split_ws_.p;
}

void HipBackend::gemm(const DeviceMatrix& W, const std::uint16_t* x, float* y, int T, float beta) {
  if (!W.i8.p) return gemm_f16(W.f16.p, x, y, T, W.K, W.N, beta);
  // int8 (measured at Llama-3-8B shapes): the GEMV up to 16 tokens; the split-K int8 GEMM
  // at 17-64 tokens on wide or long-K matrices; the GEMV up to 64 tokens on narrower ones;
  // above 64 tokens the large-tile int8 GEMM with its K split (T = 560: 370 us per
  // Llama-3-8B layer against 455 us for dequantize + library GEMM, relay's path for every
  // T above its GEMV limit). Dequantize + library GEMM remains only for K not a multiple
  // of 64.
  // 17-64 tokens on wide or long-K matrices: the int8 GEMM with the 32- or 64-token tile and
  // K cut into ranges (T = 32: Llama-3-8B gate_up 32.8 us, down 24.3; TinyLlama gate_up 15.0
  // against 15.7 for the GEMV, down 12.3 against 15.2); the GEMV stays ahead on matrices of
  // K <= 4096 and <= 6144 rows (4096 x 4096 at T = 32: 12.5 against 13.5 us).
  if (T > 16 && T <= 64 && W.K % 64 == 0 && W.N % 4 == 0 && (W.N >= 8192 || W.K >= 5000)) {
    const int ks = rh_gemm_w8_split_plan(T, W.K, W.N);
    RH_CHECK(rh_gemm_w8_skinny(W.i8.p, W.ldw, W.scale.p, x, y, T, W.K, W.N, beta, ks, w8_split_ws(ks, T, W.N), stream_));
    return;
  }
  if (T <= rh_gemv_int8_max_tokens()) {
    RH_CHECK(rh_gemv_int8(W.i8.p, W.ldw, W.scale.p, 0, x, y, T, W.K, W.N, beta, stream_));
    return;
  }
  if (W.K % 64 == 0) {
    const int ks = rh_gemm_w8_plan(T, W.K, W.N);
    RH_CHECK(rh_gemm_w8_split(W.i8.p, W.ldw, W.scale.p, x, y, T, W.K, W.N, beta, ks, w8_split_ws(ks, T, W.N), stream_));
    return;
  }
  RH_CHECK(rh_dequant_int8(W.i8.p, W.ldw, W.scale.p, W.N, W.K, dequant_.p, stream_));
  gemm_f16(dequant_.p, x, y, T, W.K, W.N, beta);
}

std::vector<float> HipBackend::forward(const ForwardBatch& batch, LayerObserver* observer) {
  const std::size_t n = enqueue_forward(batch, observer, std::numeric_limits<std::size_t>::max());
  std::vector<float> out(n);
  finish_forward(out.data(), n);
  return out;
}

int HipBackend::forward_into(const ForwardBatch& batch, float* dst, std::size_t cap) {
  const std::size_t n = enqueue_forward(batch, nullptr, cap);
  finish_forward(dst, n);
  return static_cast<int>(n / c_.vocab);
}

std::size_t HipBackend::enqueue_forward(const ForwardBatch& batch, LayerObserver* observer, std::size_t cap) {
  HIP_CHECK(hipSetDevice(device_));  // the caller's current device may be another GPU
  const int H = c_.hidden, Q = c_.q_dim(), I = c_.intermediate, D = c_.head_dim, V = c_.vocab;
  const int QKV = Q + 2 * c_.kv_dim();

  // Flatten (cuda_backend.cu:508-527).
  std::vector<int> tok, pos, seq, table_off, tables, rows, decode;
  std::vector<int> pf_t0, pf_rows, pf_pos0, pf_toff;  // prefill chunks
  const int S = static_cast<int>(batch.seqs.size());
  int max_ctx = 0;
  for (int s = 0; s < S; ++s) {
    const SeqChunk& ch = batch.seqs[s];
    const int n = static_cast<int>(ch.tokens.size());
    const int end = ch.start_pos + n;
    if (static_cast<int>(ch.block_table.size()) < layout_.blocks_for(end))
      throw std::invalid_argument("block table too short");
    if (end > max_context_) throw std::invalid_argument("sequence longer than max_context");
    for (int b : ch.block_table)
      if (b < 0 || b >= layout_.num_blocks) throw std::invalid_argument("block id outside the cache");
    table_off.push_back(static_cast<int>(tables.size()));
    tables.insert(tables.end(), ch.block_table.begin(), ch.block_table.end());
    const int t0 = static_cast<int>(tok.size());
    for (int i = 0; i < n; ++i) {
      if (ch.tokens[i] < 0 || ch.tokens[i] >= V) throw std::out_of_range("token id out of range");
      if (batch.all_logits) rows.push_back(t0 + i);
      tok.push_back(ch.tokens[i]);
      pos.push_back(ch.start_pos + i);
      seq.push_back(s);
    }
    // An empty chunk has no last row to take logits from; relay's backends would read the
    // row before it (cuda_backend.cu:523, cpu_backend.cpp:205-206: row -1 for a leading
    // one), so it is rejected instead of answered with an unrelated row.
    if (!batch.all_logits && ch.want_logits && n == 0)
      throw std::invalid_argument("a chunk with no tokens cannot want logits");
    if (!batch.all_logits && ch.want_logits) rows.push_back(t0 + n - 1);
    // Routing: one token -> decode; more -> prefill.
    if (n == 1) {
      // (token row, context length, block-table offset): the decode kernel's descriptor
      decode.insert(decode.end(), {t0, end, table_off.back(), 0});
      max_ctx = std::max(max_ctx, end);
    } else {
      pf_t0.push_back(t0);
      pf_rows.push_back(n);
      pf_pos0.push_back(ch.start_pos);
      pf_toff.push_back(table_off.back());
    }
  }
  const int T = static_cast<int>(tok.size()), R = static_cast<int>(rows.size());
  if (T == 0) return 0;
  if (T > max_tokens_) throw std::invalid_argument("batch has more tokens than max_batch_tokens");
  if (static_cast<std::size_t>(R) * V > cap) throw std::invalid_argument("logits buffer too small");
  // Prefill work records (heaviest first).
  const int n_chunks = static_cast<int>(pf_t0.size());
  std::vector<int> work(8 * static_cast<std::size_t>(n_chunks + T / rh_prefill_tile_rows() + 1));
  const int n_work = n_chunks ? rh_prefill_plan(pf_t0.data(), pf_rows.data(), pf_pos0.data(), pf_toff.data(), n_chunks,
                                                c_.heads, work.data(), static_cast<int>(work.size() / 8))
                              : 0;
  if (n_work < 0) throw std::runtime_error(std::string("HIP: ") + rh_last_error());
  work.resize(8 * static_cast<std::size_t>(n_work));
  const int n_dec = static_cast<int>(decode.size() / 4);

  // One packed metadata copy.
  // The decode descriptors and prefill work records come first: 16-byte aligned.
  const std::size_t o_dec = 0, o_work = o_dec + decode.size(), o_tok = o_work + work.size(), o_pos = o_tok + T,
                    o_seq = o_pos + T, o_toff = o_seq + T, o_tab = o_toff + S, o_rows = o_tab + tables.size(),
                    total = o_rows + R;
  meta_host_.reserve(total * sizeof(int));
  int* mh = static_cast<int*>(meta_host_.p);
  auto put = [&](std::size_t off, const std::vector<int>& v) { std::copy(v.begin(), v.end(), mh + off); };
  put(o_tok, tok);
  put(o_pos, pos);
  put(o_seq, seq);
  put(o_toff, table_off);
  put(o_tab, tables);
  put(o_rows, rows);
  put(o_dec, decode);
  put(o_work, work);
  if (meta_dev_.n < total) meta_dev_ = DeviceArray<int>(total * 2);
  HIP_CHECK(hipMemcpyAsync(meta_dev_.p, mh, total * sizeof(int), hipMemcpyHostToDevice, stream_));
  const int* d_tok = meta_dev_.p + o_tok;
  const int* d_pos = meta_dev_.p + o_pos;
  const int* d_seq = meta_dev_.p + o_seq;
  const int* d_toff = meta_dev_.p + o_toff;
  const int* d_tab = meta_dev_.p + o_tab;
  const int* d_rows = meta_dev_.p + o_rows;
  const int* d_dec = meta_dev_.p + o_dec;
  const int* d_work = meta_dev_.p + o_work;

  // Keys per decode split: relay fixes 512 (cuda_kernels.cuh:190); here the planner picks
  // the split for this step's shape (results differ only by rounding).
  const int slice = fast_attention_ && n_dec
                        ? rh_decode_slice_keys(n_dec, c_.kv_heads, c_.heads / c_.kv_heads, D, max_ctx)
                        : 0;
  const int parts = n_dec && slice > 0 ? (max_ctx + slice - 1) / slice : 0;
  if (fast_attention_ && n_dec) {
    const std::size_t need = static_cast<std::size_t>(n_dec) * c_.heads * parts;
    if (need * D > part_o_.n) part_o_ = DeviceArray<float>(need * D * 2);
    if (need * 2 > part_ml_.n) part_ml_ = DeviceArray<float>(need * 4);
    const int G = c_.heads / c_.kv_heads;
    const std::size_t groups = static_cast<std::size_t>(n_dec) * c_.kv_heads * ((G + 15) / 16);
    if (groups > counters_.n) {
      counters_ = DeviceArray<int>(groups * 2);
      HIP_CHECK(hipMemsetAsync(counters_.p, 0, counters_.n * sizeof(int), stream_));
    }
  }

  const float eps = static_cast<float>(c_.rms_eps), scale = 1.0f / std::sqrt(static_cast<float>(D));
  // The fast attention kernels take q already in their exp2 domain: the q writers round
  // q * scale * log2(e) to fp16 once, and the kernels get scale = ln 2, i.e. a unit
  // multiplier (scale * log2(e) rounds to exactly 1.0f).
  const float q_scale = scale * 1.4426950408889634f, attn_scale = 0.6931471805599453f;
  HIP_CHECK(hipEventRecord(fwd_begin_, stream_));
  RH_CHECK(rh_embed(d_tok, T, embed_.p, H, x_.p, stream_));
  bool attn_xn_ready = false;  // the previous layer's fused down merge wrote this layer's xn
  for (int l = 0; l < c_.layers; ++l) {
    DeviceLayer& L = layers_[l];
    std::uint16_t* kc = kc_.p + static_cast<std::size_t>(l) * layout_.layer_elems();
    std::uint16_t* vc = vc_.p + static_cast<std::size_t>(l) * layout_.layer_elems();
    const float* bias = L.bqkv.n ? L.bqkv.p : nullptr;
    std::uint16_t* q_out = fast_attention_ ? qh_.p : nullptr;
    // int8: the RMSNorm prologue only while T x H <= 8192 (TinyLlama int8 b = 8: 1.034 ->
    // 1.015 ms with the separate RMSNorm launch; b = 4 level).
    if (fused(L.wqkv, T, true) && D % 16 == 0 && (!L.wqkv.i8.p || T * H <= 8192)) {
      // RMSNorm, the projection and qkv_post in one launch.
      if (L.wqkv.i8.p)
        RH_CHECK(rh_gemv_int8_rmsnorm_qkv(L.wqkv.i8.p, L.wqkv.ldw, L.wqkv.scale.p, 0, x_.p, L.attn_norm.p, eps, qkv_.p,
                                          T, H, bias, inv_freq_.p, d_pos, d_seq, d_toff, d_tab, kc, vc, q_out,
                                          q_scale, c_.heads, c_.kv_heads, D, layout_.block_size, stream_));
      else
        RH_CHECK(rh_gemv_f16_rmsnorm_qkv(L.wqkv.f16.p, H, x_.p, L.attn_norm.p, eps, qkv_.p, T, H, bias, inv_freq_.p,
                                         d_pos, d_seq, d_toff, d_tab, kc, vc, q_out, q_scale, c_.heads, c_.kv_heads,
                                         D, layout_.block_size, stream_));
    } else if (L.wqkv.i8.p && D % 16 == 0 && H % 16 == 0 && T <= 32 && (QKV + 15) / 16 <= 256) {
      // int8: the projection and qkv_post in one launch (its 16-row tiles in one round;
      // TinyLlama int8 b = 16 decode step 1.369 -> 1.352 ms on the 16-row tile, whose place
      // the whole-line kernel has taken).
      if (!attn_xn_ready) RH_CHECK(rh_rmsnorm(x_.p, nullptr, T, L.attn_norm.p, H, eps, xn_.p, stream_));
      RH_CHECK(rh_gemv_int8_qkv(L.wqkv.i8.p, L.wqkv.ldw, L.wqkv.scale.p, 0, xn_.p, qkv_.p, T, H, bias, inv_freq_.p,
                                d_pos, d_seq, d_toff, d_tab, kc, vc, q_out, q_scale, c_.heads, c_.kv_heads, D,
                                layout_.block_size, stream_));
    } else if (!L.wqkv.i8.p && D % 16 == 0 && H % 16 == 0 &&
               (T <= 16 || (T <= rh_gemv_f16_max_tokens() && QKV <= 4096)) && rh_gemv_f16_split_plan(T, H, QKV) == 1) {
      // (17-32 tokens: TinyLlama's 2560-row qkv 11.1 us on the 16-row tile against 9.5 + 3.0 us
      // for the library product and a separate qkv_post; the whole-line kernel since: 32 x 2048
      // decode step 1.638 -> 1.573-1.603 ms.)
      // The projection and qkv_post in one launch (the RMSNorm cannot be folded in here).
      if (!attn_xn_ready) RH_CHECK(rh_rmsnorm(x_.p, nullptr, T, L.attn_norm.p, H, eps, xn_.p, stream_));
      RH_CHECK(rh_gemv_f16_qkv(L.wqkv.f16.p, H, xn_.p, qkv_.p, T, H, bias, inv_freq_.p, d_pos, d_seq, d_toff, d_tab,
                               kc, vc, q_out, q_scale, c_.heads, c_.kv_heads, D, layout_.block_size, stream_));
    } else {
      if (!attn_xn_ready) RH_CHECK(rh_rmsnorm(x_.p, nullptr, T, L.attn_norm.p, H, eps, xn_.p, stream_));
      gemm(L.wqkv, xn_.p, qkv_.p, T, 0.0f);
      // The fast kernels read only the fp16 q and the cache; the reference kernel reads qkv.
      if (q_out)
        RH_CHECK(rh_qkv_post_to_cache(qkv_.p, T, bias, inv_freq_.p, d_pos, d_seq, d_toff, d_tab, kc, vc, q_out,
                                      q_scale, c_.heads, c_.kv_heads, D, layout_.block_size, stream_));
      else
        RH_CHECK(rh_qkv_post(qkv_.p, T, bias, inv_freq_.p, d_pos, d_seq, d_toff, d_tab, kc, vc, q_out, 1.0f,
                             c_.heads, c_.kv_heads, D, layout_.block_size, stream_));
    }
    attn_xn_ready = false;
    HIP_CHECK(hipEventRecord(layer_done_[l], stream_));
    if (observer) observer->kv_written(l);
    if (fast_attention_) {
      if (n_work)
        RH_CHECK(rh_flash_prefill(qh_.p, Q, kc, vc, d_tab, d_work, n_work, c_.heads, c_.kv_heads, D,
                                  layout_.block_size, attn_scale, attn_.p, Q, stream_));
      if (n_dec)
        RH_CHECK(rh_paged_decode_attention(qh_.p, Q, kc, vc, d_dec, d_tab, n_dec, c_.heads,
                                           c_.kv_heads, D, layout_.block_size, slice, parts, attn_scale,
                                           part_o_.p, part_ml_.p, counters_.p, attn_.p, Q, stream_));
    } else {
      RH_CHECK(rh_reference_attention(qkv_.p, QKV, kc, vc, d_pos, d_seq, d_toff, d_tab, nullptr, T, c_.heads,
                                      c_.kv_heads, D, layout_.block_size, scale, attn_.p, Q, stream_));
    }
    // int8 products split over K (17+ tokens) leave their partials to the consumer: the o
    // and down projections' merge, residual add and following RMSNorm run as one launch,
    // the gate_up merge and SiLU as another (TinyLlama int8 32 x 2048 decode step: two
    // launches fewer per layer).
    bool mlp_xn_ready = false;
    const bool merge_norm = rh_w8_merge_rmsnorm_fits(H);
    if (const int ks = merge_norm ? w8_partials(L.wo, attn_.p, T) : 0) {
      RH_CHECK(rh_w8_merge_rmsnorm(split_ws_.p, ks, T, H, L.wo.scale.p, x_.p, L.mlp_norm.p, eps, xn_.p, stream_));
      mlp_xn_ready = true;
    } else {
      gemm(L.wo, attn_.p, x_.p, T, 1.0f);  // x += attn W_o^T
    }
    bool act_ready = false;
    if (fused(L.w_gate_up, T)) {
      RH_CHECK(rh_gemv_f16_rmsnorm(L.w_gate_up.f16.p, H, x_.p, L.mlp_norm.p, eps, gu_.p, T, H, 2 * I, 0.0f,
                                   stream_));
    } else {
      // (int8 at 9-16 tokens: level at b = 12, 1.29 -> 1.305 ms at b = 16 on TinyLlama.)
      const bool i8_silu = L.w_gate_up.i8.p && T <= 8 && H % 16 == 0;
      // fp16 where gemm() would take the whole-line product: the same kernel with SiLU·mul
      // in its epilogue.
      const bool f16_silu = !L.w_gate_up.i8.p && skinny(H, 2 * I, T) && T <= 32;
      if (i8_silu && !mlp_xn_ready && rh_gemv_f16_fused_fits(T, H) && (I + 7) / 8 < 256) {
        // The RMSNorm, the int8 product and SiLU·mul in one launch, where its workgroups
        // (8 outputs each) fit one round on the CUs: every workgroup normalises x again, which
        // at more rounds costs more than the launch it saves (SmolLM2-135M int8 decode, 192
        // workgroups: 0.770 -> 0.733 ms per step; TinyLlama, 704: 0.854 -> 0.968).
        RH_CHECK(rh_gemv_int8_rmsnorm_gate_up_silu(L.w_gate_up.i8.p, L.w_gate_up.ldw, L.w_gate_up.scale.p, 0, x_.p,
                                                   L.mlp_norm.p, eps, act_.p, T, H, I, stream_));
        act_ready = true;
      } else {
        if (!mlp_xn_ready) RH_CHECK(rh_rmsnorm(x_.p, nullptr, T, L.mlp_norm.p, H, eps, xn_.p, stream_));
        // Above 64 tokens, where the plan runs gate_up unsplit on the 256 x 96 tile: the same
        // product with SiLU·mul in its epilogue (same bytes, no fp32 [T, 2 I] round trip).
        const bool tile_silu = L.w_gate_up.i8.p && T > 64 && rh_gemm_w8_plan(T, H, 2 * I) == 1 &&
                               rh_gemm_w8_kernel(T, H, 2 * I, 1) == 1 &&
                               (static_cast<std::int64_t>(I) + 256) * L.w_gate_up.ldw < (std::int64_t(1) << 31);
        const int ks = tile_silu || I % 8 ? 0 : w8_partials(L.w_gate_up, xn_.p, T);
        if (tile_silu) {
          RH_CHECK(rh_gemm_w8_gate_up_silu(L.w_gate_up.i8.p, L.w_gate_up.ldw, L.w_gate_up.scale.p, xn_.p, act_.p, T, H,
                                           I, stream_));
          act_ready = true;
        } else if (ks) {
          RH_CHECK(rh_w8_merge_silu(split_ws_.p, ks, T, I, L.w_gate_up.scale.p, act_.p, stream_));
          act_ready = true;
        } else if (i8_silu) {
          // gemm()'s product at this T (the int8 GEMV) with SiLU·mul in its epilogue: one
          // launch fewer per layer (the same bits at 1-8 tokens).
          RH_CHECK(rh_gemv_int8_gate_up_silu(L.w_gate_up.i8.p, L.w_gate_up.ldw, L.w_gate_up.scale.p, 0, xn_.p,
                                             act_.p, T, H, I, stream_));
          act_ready = true;
        } else if (f16_silu) {
          RH_CHECK(rh_gemv_f16_gate_up_silu(L.w_gate_up.f16.p, H, xn_.p, act_.p, T, H, I, stream_));
          act_ready = true;
        } else {
          gemm(L.w_gate_up, xn_.p, gu_.p, T, 0.0f);
        }
      }
    }
    // The SiLU prologue computes T x I activations in every workgroup: only while that is
    // small (TinyLlama fp16 decode, I = 5632: b = 2 1.085 -> 1.063 ms, b = 4 1.177 -> 1.103
    // with the separate SiLU launch, level at b = 1 and 8; SmolLM2-135M, I = 1536, b = 1
    // fused: 1087 against 1048 tok/s).
    if (!act_ready && fused(L.w_down, T) && T * I <= 8192) {
      RH_CHECK(rh_gemv_f16_silu(L.w_down.f16.p, I, gu_.p, x_.p, T, I, H, 1.0f, stream_));  // x += act W_down^T
    } else {
      if (!act_ready) RH_CHECK(rh_silu_mul(gu_.p, T, I, act_.p, stream_));
      const int ks = merge_norm && l + 1 < c_.layers ? w8_partials(L.w_down, act_.p, T) : 0;
      if (ks) {  // x += act W_down^T, then the next layer's attention RMSNorm
        RH_CHECK(rh_w8_merge_rmsnorm(split_ws_.p, ks, T, H, L.w_down.scale.p, x_.p, layers_[l + 1].attn_norm.p, eps,
                                     xn_.p, stream_));
        attn_xn_ready = true;
      } else {
        gemm(L.w_down, act_.p, x_.p, T, 1.0f);  // x += act W_down^T
      }
    }
  }
  if (R) {
    RH_CHECK(rh_rmsnorm(x_.p, d_rows, R, final_norm_.p, H, eps, xn_.p, stream_));
    gemm_f16(lm_head_.n ? lm_head_.p : embed_.p, xn_.p, logits_.p, R, H, V, 0.0f);
  }
  HIP_CHECK(hipEventRecord(fwd_end_, stream_));
  pending_ = true;
  return static_cast<std::size_t>(R) * V;
}

// Runs share(j) for j = 0 .. workers - 1: share 0 on the calling thread, the others on
// helper threads (a share whose thread cannot be started runs on the calling thread). Every
// helper is joined before this returns, on every path; the first exception any share
// threw is rethrown after the join.
template <typename F>
static void run_shares(int workers, F&& share) {
  std::mutex mu;
  std::exception_ptr err;
  auto guarded = [&](int j) {
    try {
      share(j);
    } catch (...) {
      std::lock_guard<std::mutex> lock(mu);
      if (!err) err = std::current_exception();
    }
  };
  struct Joiner {
    std::vector<std::thread> t;
    ~Joiner() {
      for (auto& x : t)
        if (x.joinable()) x.join();
    }
  } helpers;
  int started = 1;
  for (int j = 1; j < workers; ++j) {
    try {
      helpers.t.emplace_back(guarded, j);
      ++started;
    } catch (const std::system_error&) {
      break;
    }
  }
  guarded(0);
  for (int j = started; j < workers; ++j) guarded(j);
  for (auto& t : helpers.t) t.join();
  if (err) std::rethrow_exception(err);
}

void HipBackend::finish_forward(float* dst, std::size_t n) {
  if (!pending_) return;
  pending_ = false;
  const std::size_t bytes = n * sizeof(float);
  std::size_t piece = 0;
  int pieces = 0;
  if (bytes) {
    logits_host_.reserve(bytes);
    if (logit_events_.empty()) {
      logit_events_.resize(kLogitChunks);
      for (auto& e : logit_events_) HIP_CHECK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    }
    piece = std::max(kLogitMinPiece, (bytes + kLogitChunks - 1) / kLogitChunks);
    piece = (piece + 255) & ~std::size_t(255);
    pieces = static_cast<int>((bytes + piece - 1) / piece);
    auto* host = static_cast<unsigned char*>(logits_host_.p);
    const auto* dev = reinterpret_cast<const unsigned char*>(logits_.p);
    for (int i = 0; i < pieces; ++i) {
      const std::size_t a = i * piece, len = std::min(piece, bytes - a);
      HIP_CHECK(hipMemcpyAsync(host + a, dev + a, len, hipMemcpyDeviceToHost, stream_));
      HIP_CHECK(hipEventRecord(logit_events_[i], stream_));
    }
  }
  HIP_CHECK(hipEventSynchronize(fwd_end_));
  float ms = 0;
  HIP_CHECK(hipEventElapsedTime(&ms, fwd_begin_, fwd_end_));
  last_ms_ = ms;
  // Large copies are split over a few host threads (one core's memcpy into freshly
  // allocated memory runs at ~10 GB/s: 25 MB of Llama-3 logits for 49 rows took ~2.5 ms).
  const auto* host = static_cast<const unsigned char*>(logits_host_.p);
  const int workers = bytes >= kLogitThreadBytes ? std::min(kLogitThreads, pieces) : 1;
  run_shares(workers, [&](int j) {
    for (int i = j; i < pieces; i += workers) {
      const std::size_t a = i * piece, len = std::min(piece, bytes - a);
      HIP_CHECK(hipEventSynchronize(logit_events_[i]));
      std::memcpy(reinterpret_cast<unsigned char*>(dst) + a, host + a, len);
    }
  });
}

// KV block traffic on the copy stream: gather into a contiguous device buffer and copy it
// to pinned host memory (and the reverse for writes), in pieces so that the host-side
// memcpy of one piece runs under the DMA of the next (one Llama-3-8B layer at 8192
// positions, 33.6 MB, into and out of caller buffers: one piece 10.9 / 20.8 GB/s read /
// write, pieces on one host thread 26.4 / 30.5, now ~37 / ~36). Serialised by copy_mu_.
void HipBackend::kv_io(int layer, const std::vector<int>& blocks, void* k_out, void* v_out, const void* k_in,
                       const void* v_in) {
  if (layer < 0 || layer >= c_.layers) throw std::invalid_argument("layer out of range");
  for (int b : blocks)
    if (b < 0 || b >= layout_.num_blocks) throw std::invalid_argument("block id outside the cache");
  const std::size_t n = blocks.size(), bb = kv_block_bytes();
  if (!n) return;
  std::lock_guard<std::mutex> lock(copy_mu_);
  const std::size_t bytes = 2 * n * bb;
  if (kv_stage_dev_.n < bytes) kv_stage_dev_ = DeviceArray<unsigned char>(bytes);
  if (kv_ids_dev_.n < n) kv_ids_dev_ = DeviceArray<int>(n);
  kv_stage_host_.reserve(bytes + n * sizeof(int));
  auto* host = static_cast<unsigned char*>(kv_stage_host_.p);
  auto* ids = reinterpret_cast<int*>(host + bytes);
  std::memcpy(ids, blocks.data(), n * sizeof(int));
  HIP_CHECK(hipMemcpyAsync(kv_ids_dev_.p, ids, n * sizeof(int), hipMemcpyHostToDevice, copy_stream_));
  const std::size_t off = static_cast<std::size_t>(layer) * layout_.layer_elems();
  if (kv_events_.empty()) {
    kv_events_.resize(kKvChunks);
    for (auto& e : kv_events_) HIP_CHECK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
  }
  // Staging bytes [0, n bb) are K, [n bb, 2 n bb) V; piece i covers [i piece, (i+1) piece).
  const int chunks = k_out ? kKvReadChunks : kKvChunks;
  const std::size_t piece = std::max<std::size_t>(kKvMinPiece, (bytes + chunks - 1) / chunks);
  const int pieces = static_cast<int>((bytes + piece - 1) / piece);
  // The host-side copies between the caller's buffers and the pinned staging run on a few
  // threads (one core moves ~10-25 GB/s; the DMA runs at the PCIe rate).
  const int workers = bytes >= kLogitThreadBytes ? std::min(kKvThreads, pieces) : 1;
  auto user_copy = [&](std::size_t a, std::size_t len, bool to_user) {
    // [a, a + len) of the staging buffer to / from k_out|k_in and v_out|v_in.
    while (len) {
      const bool is_k = a < n * bb;
      const std::size_t rel = is_k ? a : a - n * bb, take = std::min(len, n * bb - rel);
      auto* u = static_cast<unsigned char*>(is_k ? (to_user ? k_out : const_cast<void*>(k_in))
                                                 : (to_user ? v_out : const_cast<void*>(v_in)));
      if (to_user) std::memcpy(u + rel, host + a, take);
      else std::memcpy(host + a, u + rel, take);
      a += take;
      len -= take;
    }
  };
  if (k_out) {
    RH_CHECK(rh_kv_gather(kc_.p + off, vc_.p + off, kv_ids_dev_.p, static_cast<int>(n), bb, kv_stage_dev_.p,
                          copy_stream_));
    for (int i = 0; i < pieces; ++i) {
      const std::size_t a = i * piece, len = std::min(piece, bytes - a);
      HIP_CHECK(hipMemcpyAsync(host + a, kv_stage_dev_.p + a, len, hipMemcpyDeviceToHost, copy_stream_));
      HIP_CHECK(hipEventRecord(kv_events_[i], copy_stream_));
    }
    // Every thread copies its share of every piece as the piece lands, so the copy after
    // the last DMA is a share of one piece, not a whole piece on one thread.
    run_shares(workers, [&](int j) {
      for (int i = 0; i < pieces; ++i) {
        HIP_CHECK(hipEventSynchronize(kv_events_[i]));
        const std::size_t a = i * piece, len = std::min(piece, bytes - a);
        auto cut = [&](int k) { return k == workers ? len : std::min(len, (len * k / workers + 4095) & ~std::size_t(4095)); };
        user_copy(a + cut(j), cut(j + 1) - cut(j), true);
      }
    });
  } else {
    // Each share copies its pieces into the staging buffer and queues their uploads (the
    // scatter below runs after every share's uploads are queued).
    run_shares(workers, [&](int j) {
      for (int i = j; i < pieces; i += workers) {
        const std::size_t a = i * piece, len = std::min(piece, bytes - a);
        user_copy(a, len, false);
        HIP_CHECK(hipMemcpyAsync(kv_stage_dev_.p + a, host + a, len, hipMemcpyHostToDevice, copy_stream_));
      }
    });
    RH_CHECK(rh_kv_scatter(kc_.p + off, vc_.p + off, kv_ids_dev_.p, static_cast<int>(n), bb, kv_stage_dev_.p,
                           copy_stream_));
    HIP_CHECK(hipStreamSynchronize(copy_stream_));
  }
}

void HipBackend::update_weight(const std::string& name, const float* src, std::size_t n) {
  HIP_CHECK(hipSetDevice(device_));
  // src may be host memory, this device's memory, or another GPU's.
  hipPointerAttribute_t attr{};
  bool on_device = false;
  int src_dev = -1;
  if (hipPointerGetAttributes(&attr, src) == hipSuccess && attr.type == hipMemoryTypeDevice) {
    on_device = true;
    src_dev = attr.device;
  } else {
    (void)hipGetLastError();
  }
  auto chunks = [&](std::size_t total, const std::function<void(const float*, std::size_t, std::size_t)>& apply) {
    if (n != total) throw std::invalid_argument("update_weight " + name + ": wrong size");
    if (on_device && src_dev == device_) {
      apply(src, 0, n);
      return;
    }
    constexpr std::size_t kStage = std::size_t(16) << 20;
    if (stage_.n < std::min(n, kStage)) stage_ = DeviceArray<float>(std::min(n, kStage));
    for (std::size_t off = 0; off < n; off += kStage) {
      const std::size_t len = std::min(kStage, n - off);
      if (on_device)
        HIP_CHECK(hipMemcpyPeerAsync(stage_.p, device_, src + off, src_dev, len * 4, stream_));
      else
        HIP_CHECK(hipMemcpyAsync(stage_.p, src + off, len * 4, hipMemcpyHostToDevice, stream_));
      apply(stage_.p, off, len);
      HIP_CHECK(hipStreamSynchronize(stream_));
    }
  };
  auto to_f16 = [&](DeviceArray<std::uint16_t>& dst) {
    chunks(dst.n, [&](const float* c, std::size_t off, std::size_t len) { RH_CHECK(rh_f32_to_f16(c, dst.p + off, len, stream_)); });
  };
  auto to_f32 = [&](DeviceArray<float>& dst) {
    chunks(dst.n, [&](const float* c, std::size_t off, std::size_t len) {
      HIP_CHECK(hipMemcpyAsync(dst.p + off, c, len * 4, hipMemcpyDeviceToDevice, stream_));
    });
  };
  auto matrix = [&](DeviceMatrix& m) {
    if (m.i8.p) throw std::logic_error("update_weight: int8 weights must be requantized; rebuild the backend");
    to_f16(m.f16);
  };
  if (name == "embed") {
    to_f16(embed_);
  } else if (name == "lm_head") {
    if (!lm_head_.n) throw std::invalid_argument("update_weight: tied embeddings have no lm_head");
    to_f16(lm_head_);
  } else if (name == "final_norm") {
    to_f32(final_norm_);
  } else if (name.rfind("layers.", 0) == 0) {
    const std::size_t dot = name.find('.', 7);
    int i = -1;
    if (dot != std::string::npos) {
      try {
        i = std::stoi(name.substr(7, dot - 7));
      } catch (const std::exception&) {
        i = -1;
      }
    }
    if (i < 0 || i >= static_cast<int>(layers_.size())) throw std::invalid_argument("update_weight: no " + name);
    DeviceLayer& L = layers_[i];
    const std::string f = name.substr(dot + 1);
    if (f == "attn_norm") to_f32(L.attn_norm);
    else if (f == "mlp_norm") to_f32(L.mlp_norm);
    else if (f == "bqkv" && L.bqkv.n) to_f32(L.bqkv);
    else if (f == "wqkv") matrix(L.wqkv);
    else if (f == "wo") matrix(L.wo);
    else if (f == "w_gate_up") matrix(L.w_gate_up);
    else if (f == "w_down") matrix(L.w_down);
    else throw std::invalid_argument("update_weight: no " + name);
  } else {
    throw std::invalid_argument("update_weight: no " + name);
  }
  HIP_CHECK(hipStreamSynchronize(stream_));
}

}  // namespace

// ---- factories ------------------------------------------------------------------------

std::unique_ptr<Backend> make_hip_backend(const HostWeights& w, int num_blocks, int block_size, int device,
                                          int max_batch_tokens, int max_context, HipOptions options) {
  const ModelConfig& c = w.config;
  std::vector<const float*> an, wq, bq, wo, mn, gu, wd;
  for (const LayerWeights& L : w.layers) {
    an.push_back(L.attn_norm.data());
    wq.push_back(L.wqkv.data());
    bq.push_back(L.bqkv.empty() ? nullptr : L.bqkv.data());
    wo.push_back(L.wo.data());
    mn.push_back(L.mlp_norm.data());
    gu.push_back(L.w_gate_up.data());
    wd.push_back(L.w_down.data());
  }
  rh_host_weights hw{w.embed.data(), w.final_norm.data(), w.lm_head.empty() ? nullptr : w.lm_head.data(),
                     an.data(), wq.data(), c.qkv_bias ? bq.data() : nullptr, wo.data(), mn.data(), gu.data(), wd.data()};
  WeightSource src;
  src.host = &hw;
  return std::make_unique<HipBackend>(c, src, num_blocks, block_size, device, max_batch_tokens, max_context, options);
}

namespace hip_detail {

Backend* new_backend(const ModelConfig& c, const rh_host_weights* hw, bool synthetic, std::uint64_t seed, float std,
                     int num_blocks, int block_size, int device, int max_tokens, int max_context, HipOptions o) {
  WeightSource src;
  src.host = hw;
  src.synthetic = synthetic;
  src.seed = seed;
  src.std = std;
  return new HipBackend(c, src, num_blocks, block_size, device, max_tokens, max_context, o);
}

int forward_into(Backend* b, const ForwardBatch& batch, float* dst, std::size_t cap) {
  return static_cast<HipBackend*>(b)->forward_into(batch, dst, cap);
}

double last_forward_ms(const Backend* b) { return static_cast<const HipBackend*>(b)->last_forward_ms(); }

void fill_kv_random(Backend* b, std::uint64_t seed, float std) { static_cast<HipBackend*>(b)->fill_kv_random(seed, std); }

}  // namespace hip_detail

}  // namespace relay
