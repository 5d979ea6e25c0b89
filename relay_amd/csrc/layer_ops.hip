// The small kernels of a transformer layer around the attention and GEMM hot spots:
// embedding lookup, RMSNorm, bias + RoPE + paged KV write, SiLU-and-multiply, KV block
// gather/scatter for transfers, fp32 -> fp16 conversion, int8 quantization, and the
// reference attention kernel. Each cites the reference kernel whose contract it keeps
// (engine/src/cuda_backend.cu). Also the C ABI's error state and device probe.
#include <cmath>
#include <string>

#include "../../include/relay_hip.h"
#include "common.h"

namespace relay_hip {

namespace {
thread_local std::string g_error;
}

void set_error(const std::string& msg) { g_error = msg; }

namespace {

constexpr int kThreads = 256;

// Sum / max over a workgroup of kThreads; `scratch` holds kThreads / 64 floats.
template <typename T>
__device__ T block_sum(T v, T* scratch) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) scratch[w] = v;
  __syncthreads();
  T r = 0;
#pragma unroll
  for (int i = 0; i < kThreads / 64; ++i) r += scratch[i];
  __syncthreads();
  return r;
}

__device__ float block_max(float v, float* scratch) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) scratch[w] = v;
  __syncthreads();
  float r = -INFINITY;
#pragma unroll
  for (int i = 0; i < kThreads / 64; ++i) r = fmaxf(r, scratch[i]);
  __syncthreads();
  return r;
}

__global__ void f32_to_f16_kernel(const float* in, half_t* out, size_t n) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    out[i] = static_cast<half_t>(in[i]);
}

// The same conversion 8 values per thread (two 16-byte loads, one 16-byte store).
__global__ void f32_to_f16_vec_kernel(const float4* in, half8* out, size_t n8) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n8;
       i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const float4 a = in[2 * i], b = in[2 * i + 1];
    out[i] = half8{static_cast<half_t>(a.x), static_cast<half_t>(a.y), static_cast<half_t>(a.z), static_cast<half_t>(a.w),
                   static_cast<half_t>(b.x), static_cast<half_t>(b.y), static_cast<half_t>(b.z), static_cast<half_t>(b.w)};
  }
}

// x[t][c] = fp32(table[tokens[t]][c]) over the flat index of x, VEC consecutive elements per
// thread and step (8 -- one 16-byte load, two 16-byte stores -- when H % 8 == 0, else 1).
template <int VEC>
__global__ void embed_kernel(const int* tokens, const half_t* table, int H, int64_t n_vec, float* x) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n_vec; i += stride) {
    const int64_t e = i * VEC;
    const int t = static_cast<int>(e / H), col = static_cast<int>(e - static_cast<int64_t>(t) * H);
    const half_t* src = table + static_cast<int64_t>(tokens[t]) * H + col;
    if (VEC == 8) {
      const half8 h = load_half8(src);
      float4* dst = reinterpret_cast<float4*>(x + e);
      dst[0] = float4{static_cast<float>(h[0]), static_cast<float>(h[1]), static_cast<float>(h[2]), static_cast<float>(h[3])};
      dst[1] = float4{static_cast<float>(h[4]), static_cast<float>(h[5]), static_cast<float>(h[6]), static_cast<float>(h[7])};
    } else {
      x[e] = static_cast<float>(*src);
    }
  }
}

// Sum of squares in double, as the fp32 CPU backend does (cpu_backend.cpp:47-52).
__global__ void rmsnorm_kernel(const float* x, const int* rows, const float* w, int H, float eps, half_t* out) {
  __shared__ double scratch[kThreads / 64];
  const int r = blockIdx.x;
  const float* xr = x + static_cast<int64_t>(rows ? rows[r] : r) * H;
  double ss = 0;
  for (int i = threadIdx.x; i < H; i += kThreads) ss += static_cast<double>(xr[i]) * xr[i];
  ss = block_sum(ss, scratch);
  const float inv = 1.0f / sqrtf(static_cast<float>(ss / H) + eps);
  for (int i = threadIdx.x; i < H; i += kThreads)
    out[static_cast<int64_t>(r) * H + i] = f16_of_product(w[i], xr[i] * inv);
}

// Rows of H <= 4 * 4 * kThreads (H % 4 == 0): every x and w load of the row is issued at
// once as float4s held in registers, then one reduction; same sum of squares in double and
// the same output expression as rmsnorm_kernel (the summation order differs).
constexpr int kRmsVec = 4;  // float4 loads per thread
__global__ void rmsnorm_vec_kernel(const float* x, const int* rows, const float* w, int H, float eps, half_t* out) {
  __shared__ double scratch[kThreads / 64];
  const int r = blockIdx.x;
  const float4* xr = reinterpret_cast<const float4*>(x + static_cast<int64_t>(rows ? rows[r] : r) * H);
  const float4* wr = reinterpret_cast<const float4*>(w);
  const int n4 = H / 4;
  float4 xv[kRmsVec], wv[kRmsVec];
#pragma unroll
  for (int i = 0; i < kRmsVec; ++i) {
    const int j = threadIdx.x + i * kThreads;
    xv[i] = j < n4 ? xr[j] : float4{0.0f, 0.0f, 0.0f, 0.0f};
    wv[i] = j < n4 ? wr[j] : float4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  double ss = 0;
#pragma unroll
  for (int i = 0; i < kRmsVec; ++i)
    ss += static_cast<double>(xv[i].x) * xv[i].x + static_cast<double>(xv[i].y) * xv[i].y +
          static_cast<double>(xv[i].z) * xv[i].z + static_cast<double>(xv[i].w) * xv[i].w;
  ss = block_sum(ss, scratch);
  const float inv = 1.0f / sqrtf(static_cast<float>(ss / H) + eps);
  half4* o = reinterpret_cast<half4*>(out + static_cast<int64_t>(r) * H);
#pragma unroll
  for (int i = 0; i < kRmsVec; ++i) {
    const int j = threadIdx.x + i * kThreads;
    if (j < n4)
      o[j] = half4{f16_of_product(wv[i].x, xv[i].x * inv),
                   f16_of_product(wv[i].y, xv[i].y * inv),
                   f16_of_product(wv[i].z, xv[i].z * inv),
                   f16_of_product(wv[i].w, xv[i].w * inv)};
  }
}

// ---- the K-range merge of a split int8 product, fused into its consumer ----------------
//
// rh_gemm_w8_partials leaves ksn raw partial planes ws[z][t][n]. The merge of a split product
// (w8_split_merge_kernel) computes y = (sum_z ws[z]) * scale (+ beta y, the ranges added in
// order); these kernels do that merge for the product's consumer in the same launch, with
// the same arithmetic, so that a decode step saves the merge launch (~4.5 us at T = 32).

constexpr int kMaxMergeSplit = 8;

// The merged, scaled values of elements (t, n .. n + 3) (beta = 0: `+ 0.0f` keeps the
// merge's sign of a zero result); every partial's 16-byte load issued before the adds.
__device__ __forceinline__ float4 merged4(const float* ws, int ksn, int64_t plane, int64_t e, const float* sc) {
  float4 p[kMaxMergeSplit];
#pragma unroll
  for (int z = 0; z < kMaxMergeSplit; ++z)
    p[z] = z < ksn ? *reinterpret_cast<const float4*>(ws + z * plane + e) : float4{0.0f, 0.0f, 0.0f, 0.0f};
  float4 v = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int z = 0; z < kMaxMergeSplit; ++z)
    if (z < ksn) v = float4{v.x + p[z].x, v.y + p[z].y, v.z + p[z].z, v.w + p[z].w};
  return float4{mul_rounded(v.x, sc[0]), mul_rounded(v.y, sc[1]), mul_rounded(v.z, sc[2]), mul_rounded(v.w, sc[3])};
}

// act = silu(gate) * up of the merged gate_up product (rows [0, I) gate, [I, 2I) up), the
// arithmetic of silu_mul_vec_kernel; 8 elements per thread.
__global__ void w8_merge_silu_kernel(const float* __restrict__ ws, int ksn, int T, int I,
                                     const float* __restrict__ scale, half_t* act) {
  const int t = blockIdx.x, i = (blockIdx.y * kThreads + threadIdx.x) * 8;
  if (i >= I) return;
  const int64_t plane = static_cast<int64_t>(T) * 2 * I, row = static_cast<int64_t>(t) * 2 * I;
  const float4 g0 = merged4(ws, ksn, plane, row + i, scale + i), g1 = merged4(ws, ksn, plane, row + i + 4, scale + i + 4);
  const float4 u0 = merged4(ws, ksn, plane, row + I + i, scale + I + i),
               u1 = merged4(ws, ksn, plane, row + I + i + 4, scale + I + i + 4);
  const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
  const float uv[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
  half8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float g = gv[e] + 0.0f, u = uv[e] + 0.0f;
    r[e] = f16_of_product(g / (1.0f + expf(-g)), u);
  }
  *reinterpret_cast<half8*>(act + static_cast<int64_t>(t) * I + i) = r;
}

// x[t] += merged product (the merge's beta = 1), then out = RMSNorm(x[t]) * w in fp16: the
// arithmetic and summation order of rmsnorm_vec_kernel (H % 4 == 0, H <= 4 kRmsVec kThreads).
__global__ void w8_merge_rmsnorm_kernel(const float* __restrict__ ws, int ksn, int T, int H,
                                        const float* __restrict__ scale, float* x, const float* __restrict__ w,
                                        float eps, half_t* out) {
  __shared__ double scratch[kThreads / 64];
  const int r = blockIdx.x;
  const int64_t plane = static_cast<int64_t>(T) * H, row = static_cast<int64_t>(r) * H;
  float4* xr = reinterpret_cast<float4*>(x + row);
  const float4* wr = reinterpret_cast<const float4*>(w);
  const int n4 = H / 4;
  float4 xv[kRmsVec], wv[kRmsVec];
#pragma unroll
  for (int i = 0; i < kRmsVec; ++i) {
    const int j = threadIdx.x + i * kThreads;
    if (j < n4) {
      const float4 old = xr[j];
      const float4 m = merged4(ws, ksn, plane, row + 4 * j, scale + 4 * j);
      xv[i] = float4{m.x + old.x, m.y + old.y, m.z + old.z, m.w + old.w};
      xr[j] = xv[i];
      wv[i] = wr[j];
    } else {
      xv[i] = wv[i] = float4{0.0f, 0.0f, 0.0f, 0.0f};
    }
  }
  double ss = 0;
#pragma unroll
  for (int i = 0; i < kRmsVec; ++i)
    ss += static_cast<double>(xv[i].x) * xv[i].x + static_cast<double>(xv[i].y) * xv[i].y +
          static_cast<double>(xv[i].z) * xv[i].z + static_cast<double>(xv[i].w) * xv[i].w;
  ss = block_sum(ss, scratch);
  const float inv = 1.0f / sqrtf(static_cast<float>(ss / H) + eps);
  half4* o = reinterpret_cast<half4*>(out + row);
#pragma unroll
  for (int i = 0; i < kRmsVec; ++i) {
    const int j = threadIdx.x + i * kThreads;
    if (j < n4)
      o[j] = half4{f16_of_product(wv[i].x, xv[i].x * inv), f16_of_product(wv[i].y, xv[i].y * inv),
                   f16_of_product(wv[i].z, xv[i].z * inv), f16_of_product(wv[i].w, xv[i].w * inv)};
  }
}

// One thread per (token, head, pair (i, i + D/2)) of every head, grid (T, pieces): bias, then
// RoPE on q and k heads, the fp32 row written back, and the fp16 copies (q to q_out, k and v
// into the paged cache). Each element is touched by one thread, so no barriers.
// WRITE_BACK: the rotated fp32 values also go back into qkv (relay's in-place semantics);
// without it only q (fp16) and the cache rows are written.
template <bool WRITE_BACK>
__global__ void qkv_post_kernel(float* qkv, const float* bias, const float* inv_freq, const int* pos, const int* seq,
                                const int* table_off, const int* tables, half_t* kc, half_t* vc, half_t* q_out,
                                float q_scale, int heads, int kv_heads, int D, int block_size) {
  const int t = blockIdx.x, half = D / 2;
  const int idx = blockIdx.y * kThreads + threadIdx.x;
  if (idx >= (heads + 2 * kv_heads) * half) return;
  const int Q = heads * D, KV = kv_heads * D, QKV = Q + 2 * KV;
  const int h = idx / half, i = idx % half;
  float* v = qkv + static_cast<int64_t>(t) * QKV + h * D;  // q heads, then k heads, then v heads
  float a = v[i], b = v[i + half];
  if (bias) {
    a += bias[h * D + i];
    b += bias[h * D + i + half];
  }
  const int p = pos[t];
  if (h < heads + kv_heads) {
    const float angle = static_cast<float>(p) * inv_freq[i];
    float sn, cs;
    sincosf(angle, &sn, &cs);
    // Products rounded before the add (no fused multiply-add), as the CPU computes them.
    const float ra = __fsub_rn(__fmul_rn(a, cs), __fmul_rn(b, sn));
    const float rb = __fadd_rn(__fmul_rn(b, cs), __fmul_rn(a, sn));
    a = ra;
    b = rb;
  }
  if (WRITE_BACK) {
    v[i] = a;
    v[i + half] = b;
  }
  if (h < heads) {
    if (q_out) {
      q_out[static_cast<int64_t>(t) * Q + h * D + i] = f16_of_product(a, q_scale);
      q_out[static_cast<int64_t>(t) * Q + h * D + i + half] = f16_of_product(b, q_scale);
    }
    return;
  }
  const int block = tables[table_off[seq[t]] + p / block_size], slot = p % block_size;
  const int kvh = (h - heads) % kv_heads;
  half_t* dst = (h < heads + kv_heads ? kc : vc) + kv_row_offset(block, kv_heads, kvh, block_size, slot, D);
  dst[i] = static_cast<half_t>(a);
  dst[i + half] = static_cast<half_t>(b);
}

__global__ void silu_mul_kernel(const float* gu, int I, half_t* act) {
  const int t = blockIdx.x;
  const float* g = gu + static_cast<int64_t>(t) * 2 * I;
  const float* u = g + I;
  for (int i = threadIdx.x; i < I; i += kThreads) {
    const float v = g[i];
    act[static_cast<int64_t>(t) * I + i] = f16_of_product(v / (1.0f + expf(-v)), u[i]);
  }
}

// 8 consecutive elements per thread, blockIdx.y over 2048-element pieces of a row (I % 8 == 0).
__global__ void silu_mul_vec_kernel(const float* gu, int I, half_t* act) {
  const int t = blockIdx.x, i = (blockIdx.y * kThreads + threadIdx.x) * 8;
  if (i >= I) return;
  const float4* g = reinterpret_cast<const float4*>(gu + static_cast<int64_t>(t) * 2 * I + i);
  const float4* u = reinterpret_cast<const float4*>(gu + static_cast<int64_t>(t) * 2 * I + I + i);
  const float4 g0 = g[0], g1 = g[1], u0 = u[0], u1 = u[1];
  const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
  const float uv[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
  half8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = f16_of_product(gv[e] / (1.0f + expf(-gv[e])), uv[e]);
  *reinterpret_cast<half8*>(act + static_cast<int64_t>(t) * I + i) = r;
}

// The K and V runs of n cache blocks against a packed buffer [K of blocks[0..n)][V of
// blocks[0..n)] (relay's transfer format): one grid-stride loop over the buffer's 16-byte
// vectors, so consecutive threads touch consecutive bytes of the buffer whatever the block
// size. TO_BUF: pools -> buffer (gather), else buffer -> pools (scatter).
template <bool TO_BUF>
__global__ void kv_pack_kernel(uint4v* k, uint4v* v, const int* blocks, int n, int64_t vecs, uint4v* buf) {
  const int64_t total = 2 * static_cast<int64_t>(n) * vecs;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < total; e += stride) {
    const int64_t piece = e / vecs;
    const bool is_v = piece >= n;
    uint4v* pool = (is_v ? v : k) + static_cast<int64_t>(blocks[is_v ? piece - n : piece]) * vecs + (e - piece * vecs);
    if (TO_BUF) buf[e] = *pool;
    else *pool = buf[e];
  }
}

// One wave per row: scale = max|w| / 127 (1 for a zero row), q = rint(w / scale).
__global__ void quantize_int8_kernel(const float* w, int N, int K, int8_t* q, int64_t ldq, float* scale) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (n >= N) return;
  const float* row = w + static_cast<int64_t>(n) * K;
  float mx = 0.0f;
  for (int k = lane; k < K; k += 64) mx = fmaxf(mx, fabsf(row[k]));
  mx = wave_max(mx);
  const float s = mx > 0.0f ? mx / 127.0f : 1.0f;
  if (lane == 0) scale[n] = s;
  for (int k = lane; k < K; k += 64) q[static_cast<int64_t>(n) * ldq + k] = static_cast<int8_t>(rintf(row[k] / s));
}

__global__ void dequant_int8_kernel(const int8_t* w8, int64_t ldw, const float* scale, int K, int64_t total,
                                    half_t* out) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t n = i / K;
    out[i] = f16_of_product(static_cast<float>(w8[n * ldw + (i - n * K)]), scale[n]);
  }
}

// 16 weights per thread: one 16-byte load of a row, two 16-byte stores (K % 16 == 0,
// ldw % 16 == 0, aligned pointers); same per-element expression as dequant_int8_kernel.
__global__ void dequant_int8_vec_kernel(const int8_t* w8, int64_t ldw, const float* scale, int K, int64_t pieces,
                                        half_t* out) {
  const int kp = K / 16;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < pieces;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t n = i / kp;
    const int k = static_cast<int>(i - n * kp) * 16;
    const uint4v q = *reinterpret_cast<const uint4v*>(w8 + n * ldw + k);
    const float sc = scale[n];
    half8 lo, hi;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      lo[e] = f16_of_product(static_cast<float>(static_cast<int8_t>(q[e / 4] >> (8 * (e % 4)))), sc);
      hi[e] = f16_of_product(static_cast<float>(static_cast<int8_t>(q[2 + e / 4] >> (8 * (e % 4)))), sc);
    }
    half8* o = reinterpret_cast<half8*>(out + n * K + k);
    o[0] = lo;
    o[1] = hi;
  }
}

// splitmix64 finalizer (Vigna), the mixing function of the synthetic-input generator.
__device__ __host__ inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

template <typename T>
__global__ void fill_normal_kernel(T* out, size_t n, uint64_t key, float mean, float std) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const uint64_t a = mix64(key + 0x9E3779B97F4A7C15ull * (2 * i + 1));
    const uint64_t b = mix64(key + 0x9E3779B97F4A7C15ull * (2 * i + 2));
    const float u1 = static_cast<float>(((a >> 11) + 1) * (1.0 / 9007199254740992.0));
    const float u2 = static_cast<float>((b >> 11) * (1.0 / 9007199254740992.0));
    const float z = sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
    out[i] = static_cast<T>(mean + std * z);
  }
}

// One workgroup per (token, head): keys in chunks of kThreads, each thread scoring one
// key in fp32, running max and sum across chunks, each thread < D accumulating one output
// dimension. fp32 q (the RoPE'd qkv rows), fp16 cache; relay's M0 kernel in role
// (cuda_backend.cu:200-243) without its context limit.
__global__ void reference_attention_kernel(const float* q, int64_t q_stride, const half_t* kc, const half_t* vc,
                                           const int* pos, const int* seq, const int* table_off, const int* tables,
                                           const int* tokens, int heads, int kv_heads, int D, int block_size,
                                           float scale, half_t* out, int64_t out_stride) {
  __shared__ float sq[256];
  __shared__ float sp[kThreads];
  __shared__ int64_t soff[kThreads];
  __shared__ float scratch[kThreads / 64];
  const int t = tokens ? tokens[blockIdx.x] : static_cast<int>(blockIdx.x);
  const int h = blockIdx.y, kvh = h / (heads / kv_heads);
  const int ctx = pos[t] + 1;
  const int* table = tables + table_off[seq[t]];
  for (int d = threadIdx.x; d < D; d += kThreads) sq[d] = q[static_cast<int64_t>(t) * q_stride + h * D + d];
  __syncthreads();
  float m = -INFINITY, l = 0.0f, acc = 0.0f;
  for (int k0 = 0; k0 < ctx; k0 += kThreads) {
    const int j = k0 + threadIdx.x;
    float s = -INFINITY;
    if (j < ctx) {
      const int64_t off = kv_row_offset(table[j / block_size], kv_heads, kvh, block_size, j % block_size, D);
      soff[threadIdx.x] = off;
      float a = 0.0f;
      for (int d = 0; d < D; ++d) a += sq[d] * static_cast<float>(kc[off + d]);
      s = a * scale;
    }
    const float cm = block_max(s, scratch);
    const float m_new = fmaxf(m, cm);
    const float alpha = m == -INFINITY ? 0.0f : expf(m - m_new);
    const float p = j < ctx ? expf(s - m_new) : 0.0f;
    sp[threadIdx.x] = p;
    const float ps = block_sum(p, scratch);  // also the barrier for sp and soff
    l = l * alpha + ps;
    m = m_new;
    if (threadIdx.x < D) {
      const int n = min(kThreads, ctx - k0);
      float a = 0.0f;
      for (int r = 0; r < n; ++r) a += sp[r] * static_cast<float>(vc[soff[r] + threadIdx.x]);
      acc = acc * alpha + a;
    }
    __syncthreads();
  }
  if (threadIdx.x < D) out[static_cast<int64_t>(t) * out_stride + h * D + threadIdx.x] = static_cast<half_t>(acc / l);
}

unsigned grid_for(size_t n) { return static_cast<unsigned>(std::min<size_t>((n + kThreads - 1) / kThreads, 8192)); }

}  // namespace
}  // namespace relay_hip

using namespace relay_hip;

extern "C" {

const char* rh_last_error(void) { return g_error.c_str(); }

int rh_device_available(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n > 0 ? 1 : 0;
}

int rh_f32_to_f16(const float* in, void* out, size_t n, void* stream) {
  if (n == 0) return 0;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  size_t done = 0;
  if ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) % 16 == 0 && n >= 8) {
    const size_t n8 = n / 8;
    RH_TRY_LAUNCH(hipLaunchKernelGGL(f32_to_f16_vec_kernel, dim3(grid_for(n8)), dim3(kThreads), 0, s,
                                     reinterpret_cast<const float4*>(in), static_cast<half8*>(out), n8));
    done = n8 * 8;
  }
  if (done < n)
    RH_TRY_LAUNCH(hipLaunchKernelGGL(f32_to_f16_kernel, dim3(grid_for(n - done)), dim3(kThreads), 0, s, in + done,
                                     static_cast<half_t*>(out) + done, n - done));
  return 0;
}

int rh_embed(const int* tokens, int T, const void* table, int H, float* x, void* stream) {
  if (T == 0) return 0;
  RH_REQUIRE(T > 0 && H > 0, "embed: bad shape");
  const int64_t n = static_cast<int64_t>(T) * H;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (H % 8 == 0 && reinterpret_cast<uintptr_t>(table) % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0) {
    RH_TRY_LAUNCH(hipLaunchKernelGGL(embed_kernel<8>, dim3(grid_for(n / 8)), dim3(kThreads), 0, s, tokens,
                                     static_cast<const half_t*>(table), H, n / 8, x));
  } else {
    RH_TRY_LAUNCH(hipLaunchKernelGGL(embed_kernel<1>, dim3(grid_for(n)), dim3(kThreads), 0, s, tokens,
                                     static_cast<const half_t*>(table), H, n, x));
  }
  return 0;
}

int rh_rmsnorm(const float* x, const int* rows, int R, const float* w, int H, float eps, void* out, void* stream) {
  if (R == 0) return 0;
  RH_REQUIRE(R > 0 && H > 0, "rmsnorm: bad shape");
  const bool vec = H % 4 == 0 && H <= 4 * kRmsVec * kThreads &&
                   (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(out)) % 16 == 0;
  RH_TRY_LAUNCH(hipLaunchKernelGGL(vec ? rmsnorm_vec_kernel : rmsnorm_kernel, dim3(R), dim3(kThreads), 0,
                                   static_cast<hipStream_t>(stream), x, rows, w, H, eps, static_cast<half_t*>(out)));
  return 0;
}

int rh_qkv_post(float* qkv, int T, const float* bias, const float* inv_freq, const int* pos, const int* seq,
                const int* table_off, const int* tables, void* kpool, void* vpool, void* q_out, float q_scale,
                int heads, int kv_heads, int head_dim, int block_size, void* stream) {
  if (T == 0) return 0;
  RH_REQUIRE(T > 0 && heads > 0 && kv_heads > 0 && head_dim > 0 && head_dim % 2 == 0 && block_size > 0,
             "qkv_post: bad shape");
  const int pairs = (heads + 2 * kv_heads) * (head_dim / 2);
  RH_TRY_LAUNCH(hipLaunchKernelGGL(qkv_post_kernel<true>, dim3(T, (pairs + kThreads - 1) / kThreads), dim3(kThreads), 0,
                                   static_cast<hipStream_t>(stream), qkv,
                                   bias, inv_freq, pos, seq, table_off, tables, static_cast<half_t*>(kpool),
                                   static_cast<half_t*>(vpool), static_cast<half_t*>(q_out), q_scale, heads, kv_heads,
                                   head_dim, block_size));
  return 0;
}

int rh_qkv_post_to_cache(const float* qkv, int T, const float* bias, const float* inv_freq, const int* pos,
                         const int* seq, const int* table_off, const int* tables, void* kpool, void* vpool,
                         void* q_out, float q_scale, int heads, int kv_heads, int head_dim, int block_size,
                         void* stream) {
  if (T == 0) return 0;
  RH_REQUIRE(T > 0 && heads > 0 && kv_heads > 0 && head_dim > 0 && head_dim % 2 == 0 && block_size > 0,
             "qkv_post_to_cache: bad shape");
  RH_REQUIRE(q_out != nullptr, "qkv_post_to_cache: q_out is required");
  const int pairs = (heads + 2 * kv_heads) * (head_dim / 2);
  RH_TRY_LAUNCH(hipLaunchKernelGGL(qkv_post_kernel<false>, dim3(T, (pairs + kThreads - 1) / kThreads), dim3(kThreads),
                                   0, static_cast<hipStream_t>(stream), const_cast<float*>(qkv), bias, inv_freq, pos,
                                   seq, table_off, tables, static_cast<half_t*>(kpool), static_cast<half_t*>(vpool),
                                   static_cast<half_t*>(q_out), q_scale, heads, kv_heads, head_dim, block_size));
  return 0;
}

int rh_silu_mul(const float* gu, int T, int I, void* act, void* stream) {
  if (T == 0) return 0;
  RH_REQUIRE(T > 0 && I > 0, "silu_mul: bad shape");
  if (I % 8 == 0 && (reinterpret_cast<uintptr_t>(gu) | reinterpret_cast<uintptr_t>(act)) % 16 == 0) {
    RH_TRY_LAUNCH(hipLaunchKernelGGL(silu_mul_vec_kernel, dim3(T, (I + 8 * kThreads - 1) / (8 * kThreads)),
                                     dim3(kThreads), 0, static_cast<hipStream_t>(stream), gu, I,
                                     static_cast<half_t*>(act)));
  } else {
    RH_TRY_LAUNCH(hipLaunchKernelGGL(silu_mul_kernel, dim3(T), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                                     gu, I, static_cast<half_t*>(act)));
  }
  return 0;
}

int rh_w8_merge_silu(const float* workspace, int ksplit, int T, int I, const float* scale, void* act, void* stream) {
  if (T == 0) return 0;
  RH_REQUIRE(T > 0 && I > 0 && I % 8 == 0 && ksplit >= 1 && ksplit <= kMaxMergeSplit,
             "w8_merge_silu: I must be a positive multiple of 8 and ksplit in 1..8");
  RH_REQUIRE(workspace && scale && act && reinterpret_cast<uintptr_t>(act) % 16 == 0, "w8_merge_silu: bad pointer");
  RH_TRY_LAUNCH(hipLaunchKernelGGL(w8_merge_silu_kernel, dim3(T, (I + 8 * kThreads - 1) / (8 * kThreads)),
                                   dim3(kThreads), 0, static_cast<hipStream_t>(stream), workspace, ksplit, T, I, scale,
                                   static_cast<half_t*>(act)));
  return 0;
}

int rh_w8_merge_rmsnorm_fits(int H) { return H > 0 && H % 4 == 0 && H <= 4 * kRmsVec * kThreads; }

int rh_w8_merge_rmsnorm(const float* workspace, int ksplit, int T, int H, const float* scale, float* x,
                        const float* norm_w, float eps, void* out, void* stream) {
  if (T == 0) return 0;
  RH_REQUIRE(T > 0 && rh_w8_merge_rmsnorm_fits(H) && ksplit >= 1 && ksplit <= kMaxMergeSplit,
             "w8_merge_rmsnorm: H must be a multiple of 4, at most 4096, and ksplit in 1..8");
  RH_REQUIRE(workspace && scale && x && norm_w && out &&
                 (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(norm_w) |
                  reinterpret_cast<uintptr_t>(out)) % 16 == 0,
             "w8_merge_rmsnorm: x, norm_w and out must be 16-byte aligned");
  RH_TRY_LAUNCH(hipLaunchKernelGGL(w8_merge_rmsnorm_kernel, dim3(T), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                                   workspace, ksplit, T, H, scale, x, norm_w, eps, static_cast<half_t*>(out)));
  return 0;
}

int rh_kv_gather(const void* kpool, const void* vpool, const int* blocks, int n, size_t block_bytes, void* buf,
                 void* stream) {
  if (n == 0) return 0;
  RH_REQUIRE(n > 0 && block_bytes % 16 == 0, "kv_gather: block bytes must be a multiple of 16");
  const int64_t vecs = static_cast<int64_t>(block_bytes / 16);
  RH_TRY_LAUNCH(hipLaunchKernelGGL(kv_pack_kernel<true>, dim3(grid_for(2 * n * vecs)), dim3(kThreads), 0,
                                   static_cast<hipStream_t>(stream), static_cast<uint4v*>(const_cast<void*>(kpool)),
                                   static_cast<uint4v*>(const_cast<void*>(vpool)), blocks, n, vecs,
                                   static_cast<uint4v*>(buf)));
  return 0;
}

int rh_kv_scatter(void* kpool, void* vpool, const int* blocks, int n, size_t block_bytes, const void* buf,
                  void* stream) {
  if (n == 0) return 0;
  RH_REQUIRE(n > 0 && block_bytes % 16 == 0, "kv_scatter: block bytes must be a multiple of 16");
  const int64_t vecs = static_cast<int64_t>(block_bytes / 16);
  RH_TRY_LAUNCH(hipLaunchKernelGGL(kv_pack_kernel<false>, dim3(grid_for(2 * n * vecs)), dim3(kThreads), 0,
                                   static_cast<hipStream_t>(stream), static_cast<uint4v*>(kpool),
                                   static_cast<uint4v*>(vpool), blocks, n, vecs,
                                   static_cast<uint4v*>(const_cast<void*>(buf))));
  return 0;
}

int rh_quantize_int8(const float* w, int N, int K, int8_t* q, int64_t ldq, float* scale, void* stream) {
  RH_REQUIRE(N > 0 && K > 0 && ldq >= K, "quantize_int8: bad shape");
  RH_TRY_LAUNCH(hipLaunchKernelGGL(quantize_int8_kernel, dim3((N + 3) / 4), dim3(kThreads), 0,
                                   static_cast<hipStream_t>(stream), w, N, K, q, ldq, scale));
  return 0;
}

int rh_dequant_int8(const int8_t* w8, int64_t ldw, const float* scale, int N, int K, void* w16, void* stream) {
  RH_REQUIRE(N > 0 && K > 0 && ldw >= K, "dequant_int8: bad shape");
  const int64_t total = static_cast<int64_t>(N) * K;
  if (K % 16 == 0 && ldw % 16 == 0 &&
      (reinterpret_cast<uintptr_t>(w8) | reinterpret_cast<uintptr_t>(w16)) % 16 == 0) {
    const int64_t pieces = total / 16;
    RH_TRY_LAUNCH(hipLaunchKernelGGL(dequant_int8_vec_kernel, dim3(grid_for(pieces)), dim3(kThreads), 0,
                                     static_cast<hipStream_t>(stream), w8, ldw, scale, K, pieces,
                                     static_cast<half_t*>(w16)));
    return 0;
  }
  RH_TRY_LAUNCH(hipLaunchKernelGGL(dequant_int8_kernel, dim3(grid_for(total)), dim3(kThreads), 0,
                                   static_cast<hipStream_t>(stream), w8, ldw, scale, K, total,
                                   static_cast<half_t*>(w16)));
  return 0;
}

int rh_fill_normal_f16(void* out, size_t n, uint64_t seed, uint64_t stream_id, float mean, float std, void* stream) {
  if (n == 0) return 0;
  const uint64_t key = mix64(seed + 0x9E3779B97F4A7C15ull * (stream_id + 1));
  RH_TRY_LAUNCH(hipLaunchKernelGGL(fill_normal_kernel<half_t>, dim3(grid_for(n)), dim3(kThreads), 0,
                                   static_cast<hipStream_t>(stream), static_cast<half_t*>(out), n, key, mean, std));
  return 0;
}

int rh_fill_normal_f32(float* out, size_t n, uint64_t seed, uint64_t stream_id, float mean, float std, void* stream) {
  if (n == 0) return 0;
  const uint64_t key = mix64(seed + 0x9E3779B97F4A7C15ull * (stream_id + 1));
  RH_TRY_LAUNCH(hipLaunchKernelGGL(fill_normal_kernel<float>, dim3(grid_for(n)), dim3(kThreads), 0,
                                   static_cast<hipStream_t>(stream), out, n, key, mean, std));
  return 0;
}

int rh_reference_attention(const float* q, int64_t q_row_stride, const void* kpool, const void* vpool,
                           const int* pos, const int* seq, const int* table_off, const int* tables,
                           const int* tokens, int n, int heads, int kv_heads, int head_dim, int block_size,
                           float scale, void* out, int64_t out_row_stride, void* stream) {
  if (n == 0) return 0;
  RH_REQUIRE(n > 0 && heads > 0 && kv_heads > 0 && heads % kv_heads == 0, "reference attention: bad head counts");
  RH_REQUIRE(head_dim > 0 && head_dim <= 256, "reference attention: head_dim must be in 1..256");
  RH_REQUIRE(block_size > 0, "reference attention: bad block size");
  RH_TRY_LAUNCH(hipLaunchKernelGGL(reference_attention_kernel, dim3(n, heads), dim3(kThreads), 0,
                                   static_cast<hipStream_t>(stream), q, q_row_stride,
                                   static_cast<const half_t*>(kpool), static_cast<const half_t*>(vpool), pos, seq,
                                   table_off, tables, tokens, heads, kv_heads, head_dim, block_size, scale,
                                   static_cast<half_t*>(out), out_row_stride));
  return 0;
}

}  // extern "C"
