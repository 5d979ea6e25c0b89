// Skinny products for decode batches on gfx950: weight-only int8 (T <= 64 tokens) and fp16
// weights (T <= 32 tokens).
//
//   y[t, n] = scale[n] * sum_k W8[n, k] * x[t, k]  (+ beta * y[t, n])       rh_gemv_int8
//   y[t, n] =            sum_k W16[n, k] * x[t, k] (+ beta * y[t, n])       rh_gemv_f16
//
// relay's gemv_int8_kernel (cuda_kernels.cuh:364-430) does the products on the vector
// ALU, once per token. Here the products run on the matrix cores instead: a 16-row tile
// of W is the A operand of v_mfma_f32_16x16x32_f16 and the tokens' activations are the
// B operand (columns = tokens), so the vector ALU only converts weights, once for all
// tokens, and the kernel stays bound by the weight stream from HBM at every T.
// At T = 1-8 an MFMA kernel with another row/k layout (gemv_int8_m8_kernel) reads whole lines
// per row instead, faster on the measured shapes.
//
// int8 -> fp16 is exact and branch-free: for a byte b, the fp16 with bits
// 0x6400 | (b ^ 0x80) is 1024 + b + 128, so subtracting 1152 leaves b (all values are
// integers below 2048, exact in fp16). Products int8 * fp16 are exact in the MFMA's fp32
// accumulation.
//
// W8 rows are ldw bytes apart. One load instruction reads 16 rows at the same k, so with
// rows exactly 4 KB apart (K = 4096) every instruction lands on the same HBM channels and
// streams ~20% slower (measured); rh_gemv_int8_row_stride pads such rows by 256 bytes.
//
// Layout of one 64-k chunk of a 16-row tile: lane (c, g) loads the 16 bytes W[n0 + c,
// k0 + 16g .. +16) -- one 16-byte load per lane, 1 KB per wave -- and splits them into the
// A operands of two MFMAs (k slots = the two 8-byte halves). Its B operands are the
// matching 32 bytes of token c's activation row (zero for c >= T). Eight (or sixteen)
// waves per workgroup split K; their 16x16 accumulators are summed in LDS in a fixed
// order, so results do not depend on timing.
//
// The fp16 kernel has the same shape: lane (c, g) loads the 32 bytes W16[n0 + c, k0 + 16g
// .. +16) of a 64-k chunk as the A operands of two MFMAs, and up to 32 tokens are two
// 16-column B blocks sharing them. It replaces the dense GEMM library call at decode batch
// sizes, where that call spends ~8 us on matrices whose weights stream in well under 1 us
// (relay uses cublasGemmEx at every T, cuda_backend.cu:726-730).
#include "../../include/relay_hip.h"
#include "common.h"

#include <algorithm>

namespace relay_hip {
namespace {

constexpr int kMaxTokens = 16;
constexpr int kMaxInt8Tokens = 64;
constexpr size_t kFusedLdsBytes = 64 << 10;  // staged activations of the fused fp16 products
constexpr int kChunk = 64;   // k per wave step
constexpr int kUnroll = 4;   // chunks whose loads are issued together

// int8 weight rows are read through a buffer resource based at the workgroup's first row
// (32-bit offsets from a scalar base instead of 64-bit addresses: measured 1-3% faster at
// T = 1-4 on the Llama-3 shapes; level for the fp16 kernel, which keeps global loads).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t weight_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7fffffff, 0x00020000);
}

__device__ __forceinline__ half8 int8x8_to_half8(uint32_t lo, uint32_t hi) {
  // bytes b -> halves with bits 0x6400 | (b ^ 0x80), minus 1152.
  const uint32_t x0 = lo ^ 0x80808080u, x1 = hi ^ 0x80808080u;
  uint32_t h[4];
  h[0] = (x0 & 0xFFu) | ((x0 & 0xFF00u) << 8) | 0x64006400u;
  h[1] = ((x0 >> 16) & 0xFFu) | ((x0 >> 8) & 0xFF0000u) | 0x64006400u;
  h[2] = (x1 & 0xFFu) | ((x1 & 0xFF00u) << 8) | 0x64006400u;
  h[3] = ((x1 >> 16) & 0xFFu) | ((x1 >> 8) & 0xFF0000u) | 0x64006400u;
  half8 v = __builtin_bit_cast(half8, uint4v{h[0], h[1], h[2], h[3]});
  const half8 bias = {1152, 1152, 1152, 1152, 1152, 1152, 1152, 1152};
  return v - bias;
}

// What the fp16 kernel's B operands are made from:
//   kPlain   x fp16 [T, K], loaded per lane;
//   kRmsNorm x fp32 [T, K] (the residual stream): fp16(w[k] * (x * 1/sqrt(mean(x^2) + eps)))
//            with the row's sum of squares in double (rmsnorm_kernel's arithmetic);
//   kSiluMul x fp32 [T, 2K] (gate | up): fp16(g / (1 + exp(-g)) * u) (silu_mul_kernel's);
// the last two are computed once per workgroup into LDS (rows K + 8 halves apart), which
// saves the separate normalisation / activation launch at decode batch sizes.
enum Prologue { kPlain = 0, kRmsNorm = 1, kSiluMul = 2 };

// What the fp16 kernel does with its sums: kStore writes y (+ beta y); kRope is the qkv
// projection's epilogue, relay's qkv_post step folded in (bias, RoPE on q and k heads,
// k and v into the paged cache as fp16, q as fp16). For kRope the tile of workgroup i
// holds rows (h D + j0 + r, h D + D/2 + j0 + r), r < 8, of head h = i / (D/16),
// j0 = 8 (i % (D/16)), so both halves of every RoPE pair end in one wave.
enum Epilogue { kStore = 0, kRope = 1, kSilu = 2 };  // kSilu: the int8 whole-line fused form only

struct RopeArgs {
  const float* bias;  // [N] or null
  const float* inv_freq;
  const int* pos;
  const int* seq;
  const int* table_off;
  const int* tables;
  half_t* kc;
  half_t* vc;
  half_t* q_out;  // [T, heads * D] or null
  float q_scale;  // q_out = fp16(fp32(q * q_scale))
  int heads, kv_heads, D, block_size;
};

// Split-K partials of the plain fp16 product: ws [ksn][T][N] fp32, one counter per 16-row
// tile (zero between launches; the merging workgroup resets it).
constexpr int kMaxSplit = 8;
struct SplitArgs {
  float* ws;
  int* counters;
};

__device__ __forceinline__ int rope_tile_row(int tile, int m, int D) {
  const int tph = D / 16, h = tile / tph, j0 = (tile - h * tph) * 8;
  return h * D + (m < 8 ? j0 + m : D / 2 + j0 + m - 8);
}

// Lane (c, g) of wave 0 holds token t's sums for tile rows m = 4g + r; the pair of row m
// (m < 8) is row m + 8, held by lane (c, g + 2). The same float operations as qkv_post
// (bias add, then a cs - b sn / b cs + a sn, products rounded, sincosf of pos * inv_freq[i]).
// The lane's bias and inverse frequencies are loaded up front (rope_operands).
__device__ __forceinline__ void rope_operands(const RopeArgs& ra, int tile, int g, float (&bias)[4],
                                              float (&ifreq)[4]) {
  const int D = ra.D, tph = D / 16, h = tile / tph, j0 = (tile - h * tph) * 8;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    bias[r] = ra.bias ? ra.bias[rope_tile_row(tile, 4 * g + r, D)] : 0.0f;
    ifreq[r] = h < ra.heads + ra.kv_heads ? ra.inv_freq[j0 + ((4 * g + r) & 7)] : 0.0f;
  }
}

__device__ __forceinline__ void rope_epilogue(const RopeArgs& ra, const float (&s)[4], const float (&bias)[4],
                                              const float (&ifreq)[4], int tile, int g, int t, bool live,
                                              float* qkv, int N, int p, int64_t kv_base) {
  const int D = ra.D, tph = D / 16, h = tile / tph, j0 = (tile - h * tph) * 8;
  const bool first = g < 2;
  float v[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) v[r] = ra.bias ? s[r] + bias[r] : s[r];
  float o[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) o[r] = __shfl_xor(v[r], 32);  // every lane takes part
  if (!live) return;
  const bool rotate = h < ra.heads + ra.kv_heads;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = 4 * g + r, j = m < 8 ? j0 + m : D / 2 + j0 + m - 8;
    float out = v[r];
    if (rotate) {
      const float angle = static_cast<float>(p) * ifreq[r];
      float sn, cs;
      sincosf(angle, &sn, &cs);
      out = first ? __fsub_rn(__fmul_rn(v[r], cs), __fmul_rn(o[r], sn))
                  : __fadd_rn(__fmul_rn(v[r], cs), __fmul_rn(o[r], sn));
    }
    qkv[static_cast<int64_t>(t) * N + h * D + j] = out;
    if (h < ra.heads) {
      if (ra.q_out) ra.q_out[static_cast<int64_t>(t) * ra.heads * D + h * D + j] = f16_of_product(out, ra.q_scale);
    } else if (h < ra.heads + ra.kv_heads) {
      ra.kc[kv_base + j] = static_cast<half_t>(out);
    } else {
      ra.vc[kv_base + j] = static_cast<half_t>(out);
    }
  }
}

// The B operands of a fused product, computed once per workgroup into LDS (sxb rows K + 8
// halves apart) by all WAVES waves: RMSNorm of x (kRmsNorm) or SiLU(gate) * up (kSiluMul).
// K is a multiple of 16 and the rows 16-byte aligned, so every thread moves whole float4
// groups, up to kStageVec of them per batch (fewer where the kernel's 128-VGPR budget of
// 16-wave workgroups would spill) with all their loads issued together: a chain of dependent load rounds here
// is latency the product waits for (the first version's element loops took ~10 us at
// T = 4, K = 5632). Ends with a barrier.

__device__ __forceinline__ void store_half4(half_t* dst, half_t a, half_t b, half_t c, half_t d) {
  *reinterpret_cast<half4*>(dst) = half4{a, b, c, d};
}

template <int PRO, int WAVES, int kStageVec>
__device__ __forceinline__ void stage_operands(const void* xin, const float* norm_w, float eps, int T, int K,
                                               half_t* sxb, float* s_inv) {
  constexpr int NT = WAVES * kWave;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int XR = K + 8, K4 = K / 4, n4 = T * K4;
  typedef float f4 __attribute__((ext_vector_type(4)));
  if (PRO == kRmsNorm) {
    const f4* x4 = static_cast<const f4*>(xin);
    const f4* w4 = reinterpret_cast<const f4*>(norm_w);
    // The first batch of staged inputs is loaded with the sums' loads (one round of loads
    // before the barrier instead of two).
    f4 vx[kStageVec], vw[kStageVec];
#pragma unroll
    for (int j = 0; j < kStageVec; ++j) {
      const int idx = threadIdx.x + j * NT;
      if (idx < n4) {
        vx[j] = x4[idx];
        vw[j] = w4[idx % K4];
      }
    }
    // Sum of squares of each row in double (rh_rmsnorm's arithmetic; the order of a double
    // sum of fp32 squares does not reach the fp32 result), one wave per row.
    for (int t = w; t < T; t += WAVES) {
      double ss = 0;
#pragma unroll 8
      for (int i = lane; i < K4; i += kWave) {
        const f4 v = x4[static_cast<int64_t>(t) * K4 + i];
        ss += static_cast<double>(v.x) * v.x + static_cast<double>(v.y) * v.y + static_cast<double>(v.z) * v.z +
              static_cast<double>(v.w) * v.w;
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
      if (lane == 0) s_inv[t] = 1.0f / sqrtf(static_cast<float>(ss / K) + eps);
    }
    __syncthreads();
    for (int b0 = 0; b0 < n4; b0 += kStageVec * NT) {
      if (b0 > 0) {
#pragma unroll
        for (int j = 0; j < kStageVec; ++j) {
          const int idx = b0 + threadIdx.x + j * NT;
          if (idx < n4) {
            vx[j] = x4[idx];
            vw[j] = w4[idx % K4];
          }
        }
      }
#pragma unroll
      for (int j = 0; j < kStageVec; ++j) {
        const int idx = b0 + threadIdx.x + j * NT;
        if (idx < n4) {
          const int t = idx / K4, i = 4 * (idx - t * K4);
          const float inv = s_inv[t];
          store_half4(sxb + t * XR + i, f16_of_product(vw[j].x, vx[j].x * inv),
                             f16_of_product(vw[j].y, vx[j].y * inv), f16_of_product(vw[j].z, vx[j].z * inv),
                             f16_of_product(vw[j].w, vx[j].w * inv));
        }
      }
    }
    __syncthreads();
  } else if (PRO == kSiluMul) {
    const f4* gu4 = static_cast<const f4*>(xin);  // [T][2 K4]: gate | up
    for (int b0 = 0; b0 < n4; b0 += kStageVec * NT) {
      f4 vg[kStageVec], vu[kStageVec];
#pragma unroll
      for (int j = 0; j < kStageVec; ++j) {
        const int idx = b0 + threadIdx.x + j * NT;
        if (idx < n4) {
          const int t = idx / K4, i = idx - t * K4;
          vg[j] = gu4[static_cast<int64_t>(t) * 2 * K4 + i];
          vu[j] = gu4[static_cast<int64_t>(t) * 2 * K4 + K4 + i];
        }
      }
#pragma unroll
      for (int j = 0; j < kStageVec; ++j) {
        const int idx = b0 + threadIdx.x + j * NT;
        if (idx < n4) {
          const int t = idx / K4, i = 4 * (idx - t * K4);
          auto act = [](float g, float u) { return f16_of_product(g / (1.0f + expf(-g)), u); };
          store_half4(sxb + t * XR + i, act(vg[j].x, vu[j].x), act(vg[j].y, vu[j].y), act(vg[j].z, vu[j].z),
                             act(vg[j].w, vu[j].w));
        }
      }
    }
    __syncthreads();
  }
}

// kRope: each token's position and (k/v tiles) paged-cache row, looked up by one wave while
// the others run the product (a chain of three dependent loads).
__device__ __forceinline__ void rope_lookups(const RopeArgs& ra, int tile, int T, int lane, int* s_pos,
                                             int64_t* s_kvrow) {
  const int tph = ra.D / 16, h = tile / tph;
  for (int t = lane; t < T; t += kWave) {
    const int p = ra.pos[t];
    s_pos[t] = p;
    if (h >= ra.heads) {
      const int block = ra.tables[ra.table_off[ra.seq[t]] + p / ra.block_size];
      s_kvrow[t] = kv_row_offset(block, ra.kv_heads, (h - ra.heads) % ra.kv_heads, ra.block_size, p % ra.block_size,
                                 ra.D);
    }
  }
}

// T <= 16 * NB tokens: NB column blocks of 16 tokens share each converted A operand, and
// RT 16-row tiles share each activation operand (a workgroup covers 16 RT rows: above 16
// tokens every workgroup re-reads all T activation rows of K through L2, so fewer, taller
// workgroups read less). Fewer chunks per load batch as NB grows keeps the operands in
// registers.
// PRO / EPI as for the fp16 kernel below (fused producer, qkv_post epilogue); a fused
// instance has NB = RT = 1 and 16-row workgroups, and issues its first batch of weight loads
// before the prologue.
template <int WAVES, int NB, int RT, bool F16_SCALE, int PRO = kPlain, int EPI = kStore>
__global__ __launch_bounds__(WAVES * kWave) void gemv_int8_kernel(const int8_t* __restrict__ w8, int64_t ldw,
                                                                  const void* __restrict__ scale,
                                                                  const void* __restrict__ xin,
                                                                  const float* __restrict__ norm_w, float eps,
                                                                  float* y, int T, int K, int N, float beta,
                                                                  int rows_per, RopeArgs ra) {
  static_assert(PRO == kPlain || (NB == 1 && RT == 1), "fused int8 products take one 16-row tile, <= 16 tokens");
  static_assert(EPI == kStore || PRO != kSiluMul, "the qkv epilogue follows a plain or RMSNorm product");
  constexpr int U = NB == 1 ? (RT <= 2 ? kUnroll : 2) : (NB == 2 ? 2 : 1);
  __shared__ float red[WAVES][RT][NB][kWave * 4];
  __shared__ float s_inv[PRO == kRmsNorm ? kMaxTokens : 1];
  __shared__ int s_pos[EPI == kRope ? NB * kMaxTokens : 1];
  __shared__ int64_t s_kvrow[EPI == kRope ? NB * kMaxTokens : 1];
  extern __shared__ __attribute__((aligned(16))) half_t sxb[];  // PRO != kPlain: [T][K + 8]
  const half_t* x = static_cast<const half_t*>(xin);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = lane & 15, g = lane >> 4;
  // Rows [n0, nl) of W: rows_per <= 16 RT rows per workgroup (the last tile may be partly
  // empty: its rows load nothing and store nothing). kRope: the tile's rows are the RoPE
  // pairs of rope_tile_row.
  const int n0 = blockIdx.x * rows_per, nl = min(N, n0 + rows_per);
  auto out_row = [&](int rt, int m) { return EPI == kRope ? rope_tile_row(blockIdx.x, m, ra.D) : n0 + 16 * rt + m; };
  const int nchunks = (K + kChunk - 1) / kChunk;
  const int per = (nchunks + WAVES - 1) / WAVES;
  const int cb = w * per, ce = min(nchunks, cb + per);
  // Rows of this workgroup lie in [row0, row0 + 16 RT) (kRope: within one head's D rows).
  const int row0 = EPI == kRope ? (blockIdx.x / (ra.D / 16)) * ra.D : n0;
  const __amdgpu_buffer_rsrc_t wrs = weight_rsrc(w8 + static_cast<int64_t>(row0) * ldw);
  int woff[RT];
  bool rv[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    woff[rt] = (min(out_row(rt, c), N - 1) - row0) * static_cast<int>(ldw);
    rv[rt] = EPI == kRope || n0 + 16 * rt + c < nl;
  }
  bool tok[NB];
  const half_t* xrow[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    tok[b] = 16 * b + c < T;
    xrow[b] = x + static_cast<int64_t>(tok[b] ? 16 * b + c : 0) * K;
  }
  const half8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
  uint4v wv[RT][U];
  auto load_w = [&](int q0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = (q0 + u) * kChunk + 16 * g;
      const bool live = q0 + u < ce && k < K;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
        wv[rt][u] = live && rv[rt] ? __builtin_amdgcn_raw_buffer_load_b128(wrs, woff[rt] + k, 0, 0) : uint4v{0u, 0u, 0u, 0u};
    }
  };
  if (PRO != kPlain) load_w(cb);

  // Wave 0 writes the results. Its row scales (and the old y for beta != 0, where the
  // registers allow) are loaded before the weights: issued after the reduction they would
  // queue behind the weight stream (measured 0.7-3.8 us of dependent-load tail).
  constexpr bool kEarlyY = NB * RT <= 2;
  float sc[RT][4], yold[RT][NB][4], rbias[4], rfreq[4];
  if (w == 0) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = min(out_row(rt, 4 * g + r), N - 1);
        if (F16_SCALE) sc[rt][r] = static_cast<float>(static_cast<const half_t*>(scale)[n]);
        else sc[rt][r] = static_cast<const float*>(scale)[n];
#pragma unroll
        for (int b = 0; b < NB; ++b)
          yold[rt][b][r] = EPI == kStore && kEarlyY && beta != 0.0f && tok[b] ? y[static_cast<int64_t>(16 * b + c) * N + n] : 0.0f;
      }
    if (EPI == kRope) rope_operands(ra, blockIdx.x, g, rbias, rfreq);
  }
  constexpr int kVec = WAVES >= 16 && PRO == kRmsNorm ? 4 : 8;
  if (PRO != kPlain) stage_operands<PRO, WAVES, kVec>(xin, norm_w, eps, T, K, sxb, s_inv);
  if (EPI == kRope && w == WAVES - 1) rope_lookups(ra, blockIdx.x, T, lane, s_pos, s_kvrow);

  float4v acc[RT][NB];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[rt][b] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
  for (int q0 = cb; q0 < ce; q0 += U) {
    if (PRO == kPlain) load_w(q0);
    half8 xa[NB][U], xb[NB][U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = (q0 + u) * kChunk + 16 * g;
      const bool live = q0 + u < ce && k < K;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (PRO == kPlain) {
          xa[b][u] = live && tok[b] ? load_half8(xrow[b] + k) : zero;
          xb[b][u] = live && tok[b] ? load_half8(xrow[b] + k + 8) : zero;
        } else {
          // Columns past T read a real row (never written out); chunks past K read nothing.
          const half_t* xs = sxb + min(16 * b + c, T - 1) * (K + 8) + k;
          xa[b][u] = live ? *reinterpret_cast<const half8*>(xs) : zero;
          xb[b][u] = live ? *reinterpret_cast<const half8*>(xs + 8) : zero;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const half8 a0 = int8x8_to_half8(wv[rt][u][0], wv[rt][u][1]);
        const half8 a1 = int8x8_to_half8(wv[rt][u][2], wv[rt][u][3]);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          acc[rt][b] = mfma16x16x32(a0, xa[b][u], acc[rt][b]);
          acc[rt][b] = mfma16x16x32(a1, xb[b][u], acc[rt][b]);
        }
      }
    if (PRO != kPlain && q0 + U < ce) load_w(q0 + U);
  }
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[w][rt][b][lane * 4 + r] = acc[rt][b][r];
  __syncthreads();
  if (w != 0) return;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      // Lane (c, g) sums the waves for token 16b + c, rows n0 + 16 rt + 4g + r, in a fixed order.
      float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ww = 0; ww < WAVES; ++ww)
#pragma unroll
        for (int r = 0; r < 4; ++r) s[r] += red[ww][rt][b][lane * 4 + r];
      if (EPI == kRope) {
        // The scaled sums as the plain product stores them, then qkv_post's arithmetic.
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = s[r] * sc[rt][r] + 0.0f;
        const int t = tok[b] ? 16 * b + c : 0;
        rope_epilogue(ra, v, rbias, rfreq, blockIdx.x, g, 16 * b + c, tok[b], y, N, s_pos[t], s_kvrow[t]);
        continue;
      }
      if (!tok[b]) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = n0 + 16 * rt + 4 * g + r;
        if (n >= nl) continue;
        float* dst = y + static_cast<int64_t>(16 * b + c) * N + n;
        *dst = s[r] * sc[rt][r] + (beta != 0.0f ? beta * (kEarlyY ? yold[rt][b][r] : *dst) : 0.0f);
      }
    }
}

// fp16 weights, T <= 16 * NB tokens (NB column blocks of 16 tokens share each A operand).
template <int WAVES, int NB, int PRO, int EPI>
__global__ __launch_bounds__(WAVES * kWave) void gemv_f16_kernel(const half_t* __restrict__ wt, int64_t ldw,
                                                                 const void* __restrict__ xin,
                                                                 const float* __restrict__ norm_w, float eps,
                                                                 float* y, int T, int K, int N, float beta,
                                                                 RopeArgs ra, SplitArgs sp) {
  // The cross-wave reduction buffer; with a prologue it reuses the staged activations' LDS
  // (after a barrier; the launcher sizes that area for both).
  __shared__ float red_static[PRO == kPlain ? WAVES * NB * kWave * 4 : 1];
  __shared__ float s_inv[2 * kMaxTokens];
  // kRope: each token's position and (k/v tiles) paged-cache row, looked up by the last wave
  // while the others run the product (a chain of three dependent loads).
  __shared__ int s_pos[EPI == kRope ? 2 * kMaxTokens : 1];
  __shared__ int64_t s_kvrow[EPI == kRope ? 2 * kMaxTokens : 1];
  extern __shared__ __attribute__((aligned(16))) half_t sxb[];  // PRO != kPlain: [T][K + 8]
  float* red = PRO == kPlain ? red_static : reinterpret_cast<float*>(sxb);
  const half_t* x = static_cast<const half_t*>(xin);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int row = EPI == kRope ? rope_tile_row(blockIdx.x, c, ra.D) : min(n0 + c, N - 1);
  // K range of this workgroup (blockIdx.y of gridDim.y), split among its waves.
  const int nchunks = (K + kChunk - 1) / kChunk;
  const int ks = blockIdx.y, ksn = gridDim.y;
  const int kc0 = ks * nchunks / ksn, kc1 = (ks + 1) * nchunks / ksn;
  const int per = (kc1 - kc0 + WAVES - 1) / WAVES;
  const int cb = kc0 + w * per, ce = min(kc1, cb + per);
  const half_t* wrow = wt + static_cast<int64_t>(row) * ldw;
  bool tok[NB];
  const half_t* xrow[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    tok[b] = 16 * b + c < T;
    xrow[b] = x + static_cast<int64_t>(tok[b] ? 16 * b + c : 0) * K;
  }
  const half8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
  const int XR = K + 8;
  // The first batch of weight loads goes out before the prologue, which does not need it.
  half8 wa[kUnroll], wb[kUnroll];
  auto load_w = [&](int q0) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int k = (q0 + u) * kChunk + 16 * g;
      const bool live = q0 + u < ce && k < K;
      wa[u] = live ? load_half8(wrow + k) : zero;
      wb[u] = live ? load_half8(wrow + k + 8) : zero;
    }
  };
  load_w(cb);
  // Wave 0's old y (beta != 0) or RoPE operands before the stream, not behind it (for one
  // token block: more would spill in the 16-wave instances).
  constexpr bool kEarlyY = NB == 1;
  float yold[NB][4], rbias[4], rfreq[4];
  if (EPI == kRope && kEarlyY && w == 0) rope_operands(ra, blockIdx.x, g, rbias, rfreq);
  if (EPI == kStore && w == 0) {
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        yold[b][r] = kEarlyY && beta != 0.0f && tok[b] ? y[static_cast<int64_t>(16 * b + c) * N + min(n0 + 4 * g + r, N - 1)] : 0.0f;
  }
  stage_operands<PRO, WAVES, WAVES >= 16 ? 4 : 8>(xin, norm_w, eps, T, K, sxb, s_inv);
  if (EPI == kRope && w == WAVES - 1) rope_lookups(ra, blockIdx.x, T, lane, s_pos, s_kvrow);

  float4v acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) acc[b] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
  for (int q0 = cb; q0 < ce; q0 += kUnroll) {
    half8 xa[NB][kUnroll], xb[NB][kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int k = (q0 + u) * kChunk + 16 * g;
      const bool live = q0 + u < ce && k < K;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (PRO == kPlain) {
          xa[b][u] = live && tok[b] ? load_half8(xrow[b] + k) : zero;
          xb[b][u] = live && tok[b] ? load_half8(xrow[b] + k + 8) : zero;
        } else {
          // Columns past T read a real row (never written out); chunks past K read nothing.
          const half_t* xs = sxb + min(16 * b + c, T - 1) * XR + k;
          xa[b][u] = live ? *reinterpret_cast<const half8*>(xs) : zero;
          xb[b][u] = live ? *reinterpret_cast<const half8*>(xs + 8) : zero;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        acc[b] = mfma16x16x32(wa[u], xa[b][u], acc[b]);
        acc[b] = mfma16x16x32(wb[u], xb[b][u], acc[b]);
      }
    if (q0 + kUnroll < ce) load_w(q0 + kUnroll);
  }
  if (PRO != kPlain) __syncthreads();  // every wave is done reading the staged activations
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[((w * NB + b) * kWave + lane) * 4 + r] = acc[b][r];
  __syncthreads();
  if (w != 0) return;
  // Lane (c, g) sums the waves for token 16b + c, rows n0 + 4g + r, in a fixed order.
  auto wave_sum = [&](int b, float (&v)[4]) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      v[r] = 0.0f;
#pragma unroll
      for (int ww = 0; ww < WAVES; ++ww) v[r] += red[((ww * NB + b) * kWave + lane) * 4 + r];
    }
  };
  if (EPI == kRope) {
    if (!kEarlyY) rope_operands(ra, blockIdx.x, g, rbias, rfreq);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      float v[4];
      wave_sum(b, v);
      const int t = tok[b] ? 16 * b + c : 0;
      rope_epilogue(ra, v, rbias, rfreq, blockIdx.x, g, 16 * b + c, tok[b], y, N, s_pos[t], s_kvrow[t]);
    }
    return;
  }
  float sum[NB][4];
#pragma unroll
  for (int b = 0; b < NB; ++b) wave_sum(b, sum[b]);
  if (ksn > 1) {
    // Split K: publish this K range's sums; the last workgroup of the row tile to arrive
    // adds the ksn partials in K-range order (the same sum whichever arrives last).
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = n0 + 4 * g + r;
        if (tok[b] && n < N) coherent_store(&sp.ws[(static_cast<int64_t>(ks) * T + 16 * b + c) * N + n], sum[b][r]);
      }
    __builtin_amdgcn_s_waitcnt(0);
    int last = 0;
    if (lane == 0) {
      const int prev = __hip_atomic_fetch_add(&sp.counters[blockIdx.x], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = prev == ksn - 1;
      if (last) __hip_atomic_store(&sp.counters[blockIdx.x], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (!__shfl(last, 0)) return;
    // One token block at a time (all its partials' loads in flight together).
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      float part[kMaxSplit][4];
#pragma unroll
      for (int q = 0; q < kMaxSplit; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int n = min(n0 + 4 * g + r, N - 1), t = tok[b] ? 16 * b + c : 0;
          part[q][r] = q < ksn && q != ks ? coherent_load(&sp.ws[(static_cast<int64_t>(q) * T + t) * N + n]) : sum[b][r];
        }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v = 0.0f;
#pragma unroll
        for (int q = 0; q < kMaxSplit; ++q)
          if (q < ksn) v += part[q][r];
        sum[b][r] = v;
      }
    }
  }
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    if (!tok[b]) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = n0 + 4 * g + r;
      if (n >= N) continue;
      float* dst = y + static_cast<int64_t>(16 * b + c) * N + n;
      *dst = sum[b][r] + (beta != 0.0f ? beta * (kEarlyY ? yold[b][r] : *dst) : 0.0f);
    }
  }
}

// One to eight tokens on the matrix cores with whole-line row loads: the 16 A rows of
// v_mfma_f32_16x16x32_f16 are 8 W rows x 2 halves of a 128-k step and its 16 B columns are 8
// tokens x the same 2 halves. Lane (c, g) loads the 16 bytes W8[r0 + c / 2, k + 64 (c % 2) +
// 16 g ..+16), so one load instruction covers 8 rows x 128 contiguous bytes (the 16-row tile
// above covers 16 rows x 64 bytes), and its B operand is token c / 2's activations at the
// same k (zero past T). Of C only the blocks whose row half equals the column half are sums
// of matching products: lane (j = 2t + h, g) keeps rows 2g and 2g + 1 of half h for token t,
// a lane shuffle adds the other half, and LDS sums the WAVES waves (which split K in runs of
// 128) in a fixed order. DEPTH steps are loaded before any is used.
//
// SILU: W is the fused [gate; up] matrix of N = 2 I rows and the workgroup's 8 RT rows are
// gate rows a0 .. a0 + 3 and up rows I + a0 .. I + a0 + 3 of each 8-row group (a0 = 4 RT
// blockIdx.x + 4 rt), so one workgroup holds both halves of 4 RT outputs and writes act[t, a]
// = fp16(silu(g) * u) (fp16 [T, I]) instead of y: the values of this kernel's plain form
// followed by silu_mul_vec_kernel, bit for bit (same sums in the same order, same
// epilogue arithmetic), one launch fewer.
template <int WAVES, int DEPTH, bool F16_SCALE, int RT = 1, bool SILU = false>
__global__ __launch_bounds__(WAVES * kWave) void gemv_int8_m8_kernel(const int8_t* __restrict__ w8, int64_t ldw,
                                                                     const void* __restrict__ scale,
                                                                     const half_t* __restrict__ x, float* y, int T,
                                                                     int K, int N, float beta) {
  // RT 8-row groups per workgroup share each B operand (activation loads) through L2 once.
  __shared__ float red[WAVES][8][8 * RT];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int r = c >> 1, h = c & 1;  // A row: W row r0 + 8 rt + r, half h; B column: token r, half h
  const int r0 = blockIdx.x * 8 * RT;
  const int I = N / 2, a0 = blockIdx.x * 4 * RT;  // SILU only
  const int nsteps = (K + 127) / 128;
  const int per = (nsteps + WAVES - 1) / WAVES;
  const int s0 = w * per, s1 = min(nsteps, s0 + per);
  // Thread 8 RT t + i writes y[t, r0 + i]; its scale and old y are loaded before the weights.
  // (SILU: thread 4 RT t + j writes act[t, a0 + j].)
  const int wt = threadIdx.x / ((SILU ? 4 : 8) * RT), wj = static_cast<int>(threadIdx.x % ((SILU ? 4 : 8) * RT));
  const int wn = SILU ? a0 + wj : r0 + wj;
  const bool writer = static_cast<int>(threadIdx.x) < (SILU ? 4 : 8) * RT * T && wn < (SILU ? I : N);
  float sc = 0.0f, scu = 0.0f, yold = 0.0f;
  if (writer) {
    auto load_scale = [&](int n) {
      return F16_SCALE ? static_cast<float>(static_cast<const half_t*>(scale)[n]) : static_cast<const float*>(scale)[n];
    };
    sc = load_scale(wn);
    if (SILU) scu = load_scale(I + wn);
    if (!SILU && beta != 0.0f) yold = y[static_cast<int64_t>(wt) * N + wn];
  }
  const int8_t* wr[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int row = SILU ? min(a0 + 4 * rt + (r & 3), I - 1) + (r >= 4 ? I : 0) : min(r0 + 8 * rt + r, N - 1);
    wr[rt] = w8 + static_cast<int64_t>(row) * ldw + 64 * h + 16 * g;
  }
  const bool tok = r < T;
  const half_t* xr = x + static_cast<int64_t>(tok ? r : 0) * K + 64 * h + 16 * g;
  const half8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
  float4v acc[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) acc[rt] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
  for (int st = s0; st < s1; st += DEPTH) {
    uint4v wv[DEPTH][RT];
    half8 xa[DEPTH], xb[DEPTH];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      const int k = (st + d) * 128 + 64 * h + 16 * g;
      const bool live = st + d < s1 && k < K;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
        wv[d][rt] = live ? *reinterpret_cast<const uint4v*>(wr[rt] + (st + d) * 128) : uint4v{0u, 0u, 0u, 0u};
      xa[d] = live && tok ? load_half8(xr + (st + d) * 128) : zero;
      xb[d] = live && tok ? load_half8(xr + (st + d) * 128 + 8) : zero;
    }
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        acc[rt] = mfma16x16x32(int8x8_to_half8(wv[d][rt][0], wv[d][rt][1]), xa[d], acc[rt]);
        acc[rt] = mfma16x16x32(int8x8_to_half8(wv[d][rt][2], wv[d][rt][3]), xb[d], acc[rt]);
      }
  }
  // Lane (column 2t + h, g) holds C rows 4g + q = (W row 2g + q / 2, half q % 2).
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const float m0 = h ? acc[rt][1] : acc[rt][0], m1 = h ? acc[rt][3] : acc[rt][2];
    const float v0 = m0 + __shfl_xor(m0, 1), v1 = m1 + __shfl_xor(m1, 1);
    if (h == 0 && tok) {
      red[w][r][8 * rt + 2 * g] = v0;
      red[w][r][8 * rt + 2 * g + 1] = v1;
    }
  }
  __syncthreads();
  if (writer) {
    if constexpr (SILU) {
      const int gi = 8 * (wj / 4) + (wj % 4);  // the gate row's slot; the up row's is gi + 4
      float vg = 0.0f, vu = 0.0f;
#pragma unroll
      for (int ww = 0; ww < WAVES; ++ww) vg += red[ww][wt][gi];
#pragma unroll
      for (int ww = 0; ww < WAVES; ++ww) vu += red[ww][wt][gi + 4];
      const float gate = vg * sc + 0.0f, up = vu * scu + 0.0f;  // the plain form's y values
      reinterpret_cast<half_t*>(y)[static_cast<int64_t>(wt) * I + wn] = f16_of_product(gate / (1.0f + expf(-gate)), up);
    } else {
      float v = 0.0f;
#pragma unroll
      for (int ww = 0; ww < WAVES; ++ww) v += red[ww][wt][wj];
      y[static_cast<int64_t>(wt) * N + wn] = v * sc + (beta != 0.0f ? beta * yold : 0.0f);
    }
  }
}

// gemv_int8_m8_kernel, 8 waves of 2 steps, 8 rows per workgroup at 1-3 tokens on every shape
// and at 4-8 where K or N is at most 2048, else 16 (T = 4: 4096 -> 14336 16.0 -> 13.6 us,
// 14336 -> 4096 15.3 -> 14.2, 4096 x 4096 6.1 -> 6.4). Measured (us, 16-row tile -> this): T = 1 4096 x 4096 7.4 -> 5.3, 4096 ->
// 14336 16.3 -> 13.1, 14336 -> 4096 16.2 -> 13.1, 2048 -> 11264 8.5 -> 6.8 (a vector-ALU
// kernel with 8 lanes per 128-byte row run and v_dot2_f32_f16 took 5.6-6.4, 14.2, 13.9, 7.7); T = 2 4096 x 4096 7.6 ->
// 5.7, 4096 -> 14336 16.7 -> 13.4, 14336 -> 4096 17.6 -> 13.4, 5632 -> 2048 6.2 -> 5.5 (the
// vector-ALU kernel's two-token form: 6.9, 17.4, -, 5.5); T = 4 4096 x 4096 7.8 -> 6.2,
// 4096 -> 1024 6.8 -> 4.5, 4096 -> 14336 16.6 -> 15.6, 2048 -> 11264 9.7 -> 7.4, 5632 ->
// 2048 8.9 -> 5.6; T = 8 4096 -> 1024 7.4 -> 4.8, 2048 -> 11264 10.2 -> 9.5, 5632 -> 2048
// 9.7 -> 6.0. At 5-8 tokens with K and N above 2048 each 8-row workgroup re-reads all
// T activation rows (twice the weight bytes through L2 at T = 8: 4096 x 4096 7.6 -> 7.9, the
// 58.7 MB matrices 18.0 -> 19.9), so those take two 8-row groups per workgroup sharing the
// activations (RT = 2): T = 8 4096 x 4096 7.5 -> 6.6, 4096 -> 14336 17.7 -> 16.5, 14336 ->
// 4096 17.7 -> 14.6.
bool m8_takes(int T, int K, int N) { return T >= 1 && T <= 8 && (T <= 3 || std::min(K, N) <= 2048); }

// 8-row workgroups that fit one round on the CUs run 16 waves of one step each: twice the
// waves over the same K, every load of a wave issued at once (us, 8 x 2 -> 16 x 1, same
// process: 4096 -> 1024 at T = 1 / 4 / 8 4.2 -> 4.1, 4.5 -> 4.3, 4.9 -> 4.7; 5632 -> 2048 at
// T = 1 5.4 -> 5.1; 2048 x 2048 4.2 -> 4.2). With more workgroups than CUs 16 waves were
// slower (4096 -> 14336 at T = 8 in 8-row groups: 20.5 against 21.5 at 8 x 2, both far
// behind the 32-row form's 15.1).
bool m8_one_round(int N) { return (N + 7) / 8 <= 256; }

template <int NB, int RT, bool F16_SCALE>
int launch_nb(const int8_t* w8, int64_t ldw, const void* scale, const half_t* x, float* y, int T, int K, int N,
              float beta, hipStream_t s, int rows_per = 16 * RT) {
  const int tiles = (N + rows_per - 1) / rows_per;
  if (tiles < 256) {
    RH_TRY_LAUNCH(hipLaunchKernelGGL((gemv_int8_kernel<16, NB, RT, F16_SCALE>), dim3(tiles), dim3(16 * kWave), 0, s,
                                     w8, ldw, scale, x, nullptr, 0.0f, y, T, K, N, beta, rows_per, RopeArgs{}));
  } else {
    RH_TRY_LAUNCH(hipLaunchKernelGGL((gemv_int8_kernel<8, NB, RT, F16_SCALE>), dim3(tiles), dim3(8 * kWave), 0, s,
                                     w8, ldw, scale, x, nullptr, 0.0f, y, T, K, N, beta, rows_per, RopeArgs{}));
  }
  return 0;
}

// Rows per workgroup that split n rows evenly over whole rounds of 256 workgroups (one per
// CU), each at most `cap` rows: ceil(n / (256 k)) for the smallest such k.
int even_rows(int n, int cap) {
  const int k = (n + 256 * cap - 1) / (256 * cap);
  return (n + 256 * k - 1) / (256 * k);
}

// gemv_int8_m8_kernel's SiLU form with the row grouping launch() below gives the plain
// product at this T (same sums); only where launch() takes that kernel (T <= 8).
template <bool F16_SCALE>
int launch_m8_silu(const int8_t* w8, int64_t ldw, const void* scale, const half_t* x, half_t* act, int T, int K,
                   int I, hipStream_t s) {
  const int N = 2 * I;
  float* out = reinterpret_cast<float*>(act);
  if (m8_takes(T, K, N) && m8_one_round(N)) {
    RH_TRY_LAUNCH(hipLaunchKernelGGL((gemv_int8_m8_kernel<16, 1, F16_SCALE, 1, true>), dim3((I + 3) / 4),
                                     dim3(16 * kWave), 0, s, w8, ldw, scale, x, out, T, K, N, 0.0f));
  } else if (m8_takes(T, K, N)) {
    RH_TRY_LAUNCH(hipLaunchKernelGGL((gemv_int8_m8_kernel<8, 2, F16_SCALE, 1, true>), dim3((I + 3) / 4),
                                     dim3(8 * kWave), 0, s, w8, ldw, scale, x, out, T, K, N, 0.0f));
  } else if (T >= 5 && N >= 14336) {
    RH_TRY_LAUNCH(hipLaunchKernelGGL((gemv_int8_m8_kernel<8, 2, F16_SCALE, 4, true>), dim3((I + 15) / 16),
                                     dim3(8 * kWave), 0, s, w8, ldw, scale, x, out, T, K, N, 0.0f));
  } else {
    RH_TRY_LAUNCH(hipLaunchKernelGGL((gemv_int8_m8_kernel<8, 2, F16_SCALE, 2, true>), dim3((I + 7) / 8),
                                     dim3(8 * kWave), 0, s, w8, ldw, scale, x, out, T, K, N, 0.0f));
  }
  return 0;
}

template <bool W16, bool F16_SCALE, int PRO, int EPI>
int launch_whole_line(const void* w, int64_t ldw, const void* scale, const void* x, const float* norm_w, float eps,
                      float* y, int T, int K, int N, float beta, hipStream_t s, const RopeArgs& ra);

template <bool F16_SCALE>
int launch(const int8_t* w8, int64_t ldw, const void* scale, const half_t* x, float* y, int T, int K, int N,
           float beta, hipStream_t s) {
  if (T >= 9 && T <= 16 && N <= 6144)  // 9-16 tokens on up to 6144 rows: the whole-line kernel
    return launch_whole_line<false, F16_SCALE, kPlain, kStore>(w8, ldw, scale, x, nullptr, 0.0f, y, T, K, N, beta, s,
                                                                RopeArgs{});
  if (m8_takes(T, K, N)) {
    if (m8_one_round(N)) {
      RH_TRY_LAUNCH(hipLaunchKernelGGL((gemv_int8_m8_kernel<16, 1, F16_SCALE>), dim3((N + 7) / 8), dim3(16 * kWave), 0,
                                       s, w8, ldw, scale, x, y, T, K, N, beta));
    } else {
      RH_TRY_LAUNCH(hipLaunchKernelGGL((gemv_int8_m8_kernel<8, 2, F16_SCALE>), dim3((N + 7) / 8), dim3(8 * kWave), 0, s,
                                       w8, ldw, scale, x, y, T, K, N, beta));
    }
    return 0;
  }
  if (T >= 5 && T <= 8 && N >= 14336) {
    // 32 rows per workgroup: a quarter of the 8-row form's activation reads through L2
    // (measured at T = 4 and 8 on Llama-3-8B's gate_up shape: L1 -> L2 read requests 1.5x
    // those at T = 1, i.e. ~0.6x the weight bytes again in activations, with 16 rows).
    // 4096 -> 14336 at T = 8 16.5 -> 15.4 us; at T = 4, or on matrices of 4096-14336 rows
    // with K = 14336 (fewer than 448 workgroups), slower.
    RH_TRY_LAUNCH(hipLaunchKernelGGL((gemv_int8_m8_kernel<8, 2, F16_SCALE, 4>), dim3((N + 31) / 32), dim3(8 * kWave), 0,
                                     s, w8, ldw, scale, x, y, T, K, N, beta));
    return 0;
  }
  if (T <= 8) {  // 16 rows per workgroup: half the activation reads of the 8-row form
    RH_TRY_LAUNCH(hipLaunchKernelGGL((gemv_int8_m8_kernel<8, 2, F16_SCALE, 2>), dim3((N + 15) / 16), dim3(8 * kWave), 0,
                                     s, w8, ldw, scale, x, y, T, K, N, beta));
    return 0;
  }
  // Two row tiles per workgroup (sharing the activation operands, half the activation
  // traffic through L2) only while that still leaves >= 192 workgroups: measured at T = 17-64,
  // N = 6144 gains up to 30% and N = 4096 with 128 workgroups loses as much; at T = 4-16 on
  // N = 14336, 17.1 -> 16.5 us (T = 4), 19.6 -> 17.8 (8), 26.0 -> 20.9 (16), while at T <= 2
  // or on N <= 4096 it is level or slower.
  const bool tall = (N + 31) / 32 >= 192;
  // More row tiles than CUs: rows are split evenly over whole rounds of 256 workgroups
  // (14336 rows in 896 tiles left half the CUs one tile more than the others: 15.0 us at
  // T = 1, 12288 rows in 768 tiles took 11.6). Measured on 4096-column matrices (us):
  // T = 1: 14-row workgroups at N = 14336 15.0 -> 14.4, 12-row at N = 6144 9.1 -> 8.6;
  // T = 4-8: the two-tile workgroups, N = 14336 16.6 -> 15.5 (T = 4), 17.9 -> 17.0 (8), N =
  // 6144 10.1 -> 8.8 (4); T = 9-16: up to four tiles in 8-row steps (one round), N = 12288
  // 18.8 -> 15.1, 14336 21.0 -> 18.3, 28672 32.1 -> 28.0 at T = 16.
  if (T <= 16 && (N + 15) / 16 > 256) {
    if (T >= 9) {
      const int units = (N + 7) / 8, m = (units + 2047) / 2048;  // rounds of 256: <= 64 rows each
      const int rows_per = 8 * ((units + 256 * m - 1) / (256 * m));
      switch ((rows_per + 15) / 16) {
        case 1: return launch_nb<1, 1, F16_SCALE>(w8, ldw, scale, x, y, T, K, N, beta, s, rows_per);
        case 2: return launch_nb<1, 2, F16_SCALE>(w8, ldw, scale, x, y, T, K, N, beta, s, rows_per);
        case 3: return launch_nb<1, 3, F16_SCALE>(w8, ldw, scale, x, y, T, K, N, beta, s, rows_per);
        default: return launch_nb<1, 4, F16_SCALE>(w8, ldw, scale, x, y, T, K, N, beta, s, rows_per);
      }
    }
    if (T >= 4 && tall) return launch_nb<1, 2, F16_SCALE>(w8, ldw, scale, x, y, T, K, N, beta, s, even_rows(N, 32));
    return launch_nb<1, 1, F16_SCALE>(w8, ldw, scale, x, y, T, K, N, beta, s, even_rows(N, 16));
  }
  if (T <= 16) return tall && T >= 4 ? launch_nb<1, 2, F16_SCALE>(w8, ldw, scale, x, y, T, K, N, beta, s)
                                     : launch_nb<1, 1, F16_SCALE>(w8, ldw, scale, x, y, T, K, N, beta, s);
  if (T <= 32) return tall ? launch_nb<2, 2, F16_SCALE>(w8, ldw, scale, x, y, T, K, N, beta, s)
                           : launch_nb<2, 1, F16_SCALE>(w8, ldw, scale, x, y, T, K, N, beta, s);
  if (T <= 48) return tall ? launch_nb<3, 2, F16_SCALE>(w8, ldw, scale, x, y, T, K, N, beta, s)
                           : launch_nb<3, 1, F16_SCALE>(w8, ldw, scale, x, y, T, K, N, beta, s);
  return tall ? launch_nb<4, 2, F16_SCALE>(w8, ldw, scale, x, y, T, K, N, beta, s)
              : launch_nb<4, 1, F16_SCALE>(w8, ldw, scale, x, y, T, K, N, beta, s);
}

// gemv_int8_m8_kernel's whole-line form with a fused producer and/or the qkv epilogue, for 1-8
// tokens: 16 rows per workgroup as two 8-row groups (kRope: the RoPE pairs of rope_tile_row, so
// both halves of every pair end in one workgroup), waves splitting K in runs of 128, the
// activations read as for the plain form (kPlain) or normalised once per workgroup into LDS
// (kRmsNorm, stage_operands: rows K + 8 halves apart, so the 16 lanes of a B read cover 8
// tokens x 2 halves on distinct banks). One writer thread per (token, row) sums the waves'
// partials in a fixed order; kRope writers take a pair (m, m + 8) and apply qkv_post's
// arithmetic (rope_epilogue's float operations). kSilu: W is the fused [gate; up] matrix and
// the workgroup's two 8-row groups are gate rows a0 + 4 rt .. +3 and the up rows I further
// (a0 = 8 blockIdx.x), so it writes act = fp16(silu(g) * u) for 8 outputs (fp16 [T, I]).
// W16: fp16 weights (gemv_f16_m8_kernel's layout: a step is 64 k, lane (c, g) loads the 8
// halves at k + 32 (c % 2) + 8 g, one MFMA per step and row group, no scale); a row's step
// is 128 bytes either way, so the weight addressing is shared.
// RT = 1 (kStore only): one 8-row group per workgroup, for matrices whose 16-row tiles would
// leave CUs idle.
template <int WAVES, int DEPTH, bool W16, bool F16_SCALE, int PRO, int EPI, int RT = 2, int NB = 1>
__global__ __launch_bounds__(WAVES * kWave) void gemv_int8_m8_fused_kernel(
    const void* __restrict__ wq, int64_t ldw, const void* __restrict__ scale, const void* __restrict__ xin,
    const float* __restrict__ norm_w, float eps, float* y, int T, int K, int N, float beta, RopeArgs ra) {
  static_assert(RT == 2 || (RT == 1 && EPI == kStore), "the qkv and SiLU epilogues pair rows in 16-row tiles");
  static_assert(WAVES >= 4, "the qkv and SiLU epilogues take one thread per (token, pair) for up to 32 tokens");
  constexpr int KS = W16 ? 64 : 128;  // k per step
  const int8_t* w8 = static_cast<const int8_t*>(wq);
  const int64_t ldb = W16 ? 2 * ldw : ldw;  // row stride in bytes
  __shared__ float red[WAVES][8 * NB][8 * RT];
  __shared__ float s_inv[8 * NB];
  __shared__ int s_pos[EPI == kRope ? 8 * NB : 1];
  __shared__ int64_t s_kvrow[EPI == kRope ? 8 * NB : 1];
  extern __shared__ __attribute__((aligned(16))) half_t sxb[];  // kRmsNorm: [T][K + 8]
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int r = c >> 1, h = c & 1;  // A row: row r of group rt, half h; B column: token r (+ 8 nb), half h
  const int I = N / 2, a0 = 8 * blockIdx.x;  // kSilu only
  auto out_row = [&](int rt, int m) -> int {  // m < 8: row m of group rt
    if (EPI == kSilu) return min(a0 + 4 * rt + (m & 3), I - 1) + (m >= 4 ? I : 0);
    return EPI == kRope ? rope_tile_row(blockIdx.x, 8 * rt + m, ra.D) : 8 * RT * blockIdx.x + 8 * rt + m;
  };
  const int nsteps = (K + KS - 1) / KS;
  const int per = (nsteps + WAVES - 1) / WAVES;
  const int s0 = w * per, s1 = min(nsteps, s0 + per);
  const int klane = W16 ? 32 * h + 8 * g : 64 * h + 16 * g;  // this lane's first k of a step
  const int8_t* wr[RT];  // byte addresses; a step is 128 bytes of a row for both weight types
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
    wr[rt] = w8 + static_cast<int64_t>(min(out_row(rt, r), N - 1)) * ldb + 64 * h + 16 * g;
  bool tok[NB];
  const half_t* xr[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    tok[nb] = r + 8 * nb < T;
    xr[nb] = static_cast<const half_t*>(xin) + static_cast<int64_t>(tok[nb] ? r + 8 * nb : 0) * K + klane;
  }
  const half8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
  uint4v wv[DEPTH][RT];
  auto load_w = [&](int st) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      const int k = (st + d) * KS + klane;
      const bool live = st + d < s1 && k < K;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
        wv[d][rt] = live ? *reinterpret_cast<const uint4v*>(wr[rt] + (st + d) * 128) : uint4v{0u, 0u, 0u, 0u};
    }
  };
  load_w(s0);  // the first weights are in flight under the prologue
  if (PRO != kPlain) stage_operands<PRO, WAVES, WAVES >= 16 ? 4 : 8>(xin, norm_w, eps, T, K, sxb, s_inv);
  if (EPI == kRope && w == WAVES - 1) rope_lookups(ra, blockIdx.x, T, lane, s_pos, s_kvrow);
  float4v acc[RT][NB];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[rt][nb] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
  for (int st = s0; st < s1; st += DEPTH) {
    if (st != s0) load_w(st);
    half8 xa[DEPTH][NB], xb[DEPTH][NB];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      const int k = (st + d) * KS + klane;
      const bool live = st + d < s1 && k < K;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        if (PRO == kPlain) {
          xa[d][nb] = live && tok[nb] ? load_half8(xr[nb] + (st + d) * KS) : zero;
          if (!W16) xb[d][nb] = live && tok[nb] ? load_half8(xr[nb] + (st + d) * KS + 8) : zero;
        } else {
          const half_t* xs = sxb + (tok[nb] ? r + 8 * nb : 0) * (K + 8) + k;
          xa[d][nb] = live && tok[nb] ? *reinterpret_cast<const half8*>(xs) : zero;
          if (!W16) xb[d][nb] = live && tok[nb] ? *reinterpret_cast<const half8*>(xs + 8) : zero;
        }
      }
    }
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        if (W16) {
          const half8 a = __builtin_bit_cast(half8, wv[d][rt]);
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) acc[rt][nb] = mfma16x16x32(a, xa[d][nb], acc[rt][nb]);
        } else {
          const half8 a = int8x8_to_half8(wv[d][rt][0], wv[d][rt][1]);
          const half8 b = int8x8_to_half8(wv[d][rt][2], wv[d][rt][3]);
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            acc[rt][nb] = mfma16x16x32(a, xa[d][nb], acc[rt][nb]);
            acc[rt][nb] = mfma16x16x32(b, xb[d][nb], acc[rt][nb]);
          }
        }
      }
  }
  // Lane (column 2t + h, g) holds C rows 4g + q = (row 2g + q / 2, half q % 2).
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const float m0 = h ? acc[rt][nb][1] : acc[rt][nb][0], m1 = h ? acc[rt][nb][3] : acc[rt][nb][2];
      const float v0 = m0 + __shfl_xor(m0, 1), v1 = m1 + __shfl_xor(m1, 1);
      if (h == 0 && tok[nb]) {
        red[w][r + 8 * nb][8 * rt + 2 * g] = v0;
        red[w][r + 8 * nb][8 * rt + 2 * g + 1] = v1;
      }
    }
  __syncthreads();
  auto row_scale = [&](int n) {
    return F16_SCALE ? static_cast<float>(static_cast<const half_t*>(scale)[n]) : static_cast<const float*>(scale)[n];
  };
  // The scaled sum of (token t, slot m = 8 rt + row) as the plain product stores it.
  auto value = [&](int t, int m) {
    float v = 0.0f;
#pragma unroll
    for (int ww = 0; ww < WAVES; ++ww) v += red[ww][t][m];
    return W16 ? v : v * row_scale(min(out_row(m >> 3, m & 7), N - 1));
  };
  if constexpr (EPI == kStore) {
    // One (token, row) output per thread; 8 RT T can exceed the workgroup at 17-32 tokens.
    for (int i = threadIdx.x; i < 8 * RT * T; i += WAVES * kWave) {
      const int t = i / (8 * RT), m = i % (8 * RT);
      const int n = 8 * RT * blockIdx.x + m;
      if (n < N) {
        float* dst = y + static_cast<int64_t>(t) * N + n;
        *dst = value(t, m) + (beta != 0.0f ? beta * *dst : 0.0f);
      }
    }
  } else if constexpr (EPI == kSilu) {
    // Thread (t, j) writes act[t, a0 + j]: gate slot 8 (j / 4) + j % 4, up slot 4 further
    // (gemv_int8_m8_kernel's SiLU epilogue arithmetic).
    const int t = threadIdx.x / 8, j = threadIdx.x % 8, a = a0 + j;
    if (threadIdx.x < 8 * T && a < I) {
      const int gi = 8 * (j / 4) + j % 4;
      const float gate = value(t, gi) + 0.0f, up = value(t, gi + 4) + 0.0f;
      reinterpret_cast<half_t*>(y)[static_cast<int64_t>(t) * I + a] = f16_of_product(gate / (1.0f + expf(-gate)), up);
    }
  } else {
    const int t = threadIdx.x / 8, m = threadIdx.x % 8;  // the pair (m, m + 8)
    if (threadIdx.x >= 8 * T) return;
    const int D = ra.D, tph = D / 16, hd = blockIdx.x / tph, j0 = (blockIdx.x - hd * tph) * 8;
    const int ja = j0 + m, jb = D / 2 + j0 + m;
    float a = value(t, m) + 0.0f, b = value(t, m + 8) + 0.0f;
    if (ra.bias) {
      a += ra.bias[hd * D + ja];
      b += ra.bias[hd * D + jb];
    }
    const int p = s_pos[t];
    if (hd < ra.heads + ra.kv_heads) {
      const float angle = static_cast<float>(p) * ra.inv_freq[ja];
      float sn, cs;
      sincosf(angle, &sn, &cs);
      const float ra_ = __fsub_rn(__fmul_rn(a, cs), __fmul_rn(b, sn));
      const float rb_ = __fadd_rn(__fmul_rn(b, cs), __fmul_rn(a, sn));
      a = ra_;
      b = rb_;
    }
    y[static_cast<int64_t>(t) * N + hd * D + ja] = a;
    y[static_cast<int64_t>(t) * N + hd * D + jb] = b;
    if (hd < ra.heads) {
      if (ra.q_out) {
        half_t* q = ra.q_out + static_cast<int64_t>(t) * ra.heads * D + hd * D;
        q[ja] = f16_of_product(a, ra.q_scale);
        q[jb] = f16_of_product(b, ra.q_scale);
      }
    } else {
      half_t* dst = (hd < ra.heads + ra.kv_heads ? ra.kc : ra.vc) + s_kvrow[t];
      dst[ja] = static_cast<half_t>(a);
      dst[jb] = static_cast<half_t>(b);
    }
  }
}

// The whole-line kernel at 1-16 tokens (two 8-token column blocks above 8): 8-row workgroups
// for plain stores while they fit one round on the CUs, else 16-row ones (row pairs for
// the qkv and SiLU epilogues); 16 waves below 256 workgroups, else 8. Measured at 9-16 tokens
// against the 16-row MFMA tile (us, T = 9 / 16): fp16 2048 x 2048 6.2 / 6.5 -> 4.6 / 4.8,
// 5632 -> 2048 11.3 / 13.0 -> 7.9 / 8.8, 2048 -> 11264 15.2 / 17.1 -> 13.2 / 13.6, 4096 ->
// 14336 29.8 / 34.7 -> 25.7 / 27.2, 14336 -> 4096 30.0 / 30.7 -> 25.1 / 25.8; int8 2048 x 2048
// 5.4 / 5.9 -> 4.7 / 5.1, 5632 -> 2048 9.4 / 11.0 -> 7.1 / 9.2, 2048 -> 2560 5.6 / 5.9 -> 4.8 /
// 5.4, 4096 x 4096 8.1 / 9.0 -> 7.5 / 8.6, 14336 -> 4096 19.9 / 23.6 -> 19.9 / 21.7 (int8 on
// 8192+ rows stays on its row-tile kernels: 4096 -> 14336 19.6 against 24.5 at T = 16).
template <bool W16, bool F16_SCALE, int PRO, int EPI>
int launch_whole_line(const void* w, int64_t ldw, const void* scale, const void* x, const float* norm_w, float eps,
                      float* y, int T, int K, int N, float beta, hipStream_t s, const RopeArgs& ra) {
  const size_t staged = PRO == kPlain ? 0 : static_cast<size_t>(T) * (K + 8) * sizeof(half_t);
  RH_REQUIRE(staged <= kFusedLdsBytes, "gemv: T * (K + 8) fp16 activations exceed the fused path's LDS");
  RH_REQUIRE(T >= 1 && T <= 32, "gemv: the whole-line kernel takes 1-32 tokens");
  const bool rt1 = EPI == kStore && (N + 7) / 8 <= 256;
  const int groups = rt1 ? (N + 7) / 8 : (N + 15) / 16;
  const bool w16 = rt1 || groups < 256;
#define RH_WL(WAVES, DEPTH, RTV, NBV)                                                                                  \
  RH_TRY_LAUNCH(hipLaunchKernelGGL((gemv_int8_m8_fused_kernel<WAVES, DEPTH, W16, F16_SCALE, PRO, EPI, RTV, NBV>),      \
                                   dim3(groups), dim3(WAVES * kWave), staged, s, w, ldw, scale, x, norm_w, eps, y, T, K, \
                                   N, beta, ra))
  // fp16 at 17-32 tokens: 8 waves of 2 steps whatever the grid (SmolLM2-135M 32 x 640 decode
  // step 1.206 -> 1.167 ms, TinyLlama 32 x 2048 level, against 16 waves below 256 workgroups).
#define RH_WL_NB(RTV, NBV)                                   \
  if (w16 && !(W16 && NBV >= 3)) {                           \
    if constexpr (W16) RH_WL(16, 4, RTV, NBV);               \
    else RH_WL(16, 1, RTV, NBV);                             \
  } else {                                                   \
    if constexpr (W16) RH_WL(8, (NBV <= 2 ? 4 : 2), RTV, NBV);  \
    else RH_WL(8, (NBV <= 2 ? 2 : 1), RTV, NBV);             \
  }
#define RH_WL_T(RTV)                    \
  if (T <= 8) { RH_WL_NB(RTV, 1) }      \
  else if (T <= 16) { RH_WL_NB(RTV, 2) } \
  else if (T <= 24) { RH_WL_NB(RTV, 3) } \
  else { RH_WL_NB(RTV, 4) }
  if constexpr (EPI == kStore) {
    if (rt1) {
      RH_WL_T(1)
      return 0;
    }
  }
  RH_WL_T(2)
#undef RH_WL_T
#undef RH_WL_NB
#undef RH_WL
  return 0;
}

// The int8 product with a fused producer (PRO) and/or the qkv epilogue (EPI): the whole-line
// kernel at 1-16 tokens (launch_whole_line; the SiLU producer keeps the 16-row tile), the
// 16-row tile above. Where the plain product takes another kernel or row grouping the sums
// come in another order (equal within the fp32 bound).
template <bool F16_SCALE, int PRO, int EPI>
int launch_fused(const int8_t* w8, int64_t ldw, const void* scale, const void* xin, const float* norm_w, float eps,
                 float* y, int T, int K, int N, float beta, hipStream_t s, const RopeArgs& ra) {
  const size_t staged = PRO == kPlain ? 0 : static_cast<size_t>(T) * (K + 8) * sizeof(half_t);
  RH_REQUIRE(staged <= kFusedLdsBytes, "gemv_int8: T * (K + 8) fp16 activations exceed the fused path's LDS");
  const int tiles = (N + 15) / 16;
  // 1-16 tokens without the SiLU producer, and the qkv epilogue up to 32: the whole-line form
  // (a one-token vector-ALU form behind the producers made TinyLlama int8 decode steps slower).
  if constexpr (PRO != kSiluMul) {
    if (T <= 16 || (EPI == kRope && T <= 32))
      return launch_whole_line<false, F16_SCALE, PRO, EPI>(w8, ldw, scale, xin, norm_w, eps, y, T, K, N, beta, s, ra);
  }
  if (tiles < 256) {
    RH_TRY_LAUNCH(hipLaunchKernelGGL((gemv_int8_kernel<16, 1, 1, F16_SCALE, PRO, EPI>), dim3(tiles), dim3(16 * kWave),
                                     staged, s, w8, ldw, scale, xin, norm_w, eps, y, T, K, N, beta, 16, ra));
  } else {
    RH_TRY_LAUNCH(hipLaunchKernelGGL((gemv_int8_kernel<8, 1, 1, F16_SCALE, PRO, EPI>), dim3(tiles), dim3(8 * kWave),
                                     staged, s, w8, ldw, scale, xin, norm_w, eps, y, T, K, N, beta, 16, ra));
  }
  return 0;
}

int check_int8_fused(const int8_t* w8, int64_t ldw, const void* scale, const void* x, int T, int K, int N,
                     int max_t = kMaxTokens) {
  RH_REQUIRE(T >= 1 && T <= max_t, max_t == kMaxTokens ? "gemv_int8 fused: T must be in 1..16"
                                                       : "gemv_int8 fused: T must be in 1..32");
  RH_REQUIRE(K > 0 && N > 0 && K % 16 == 0, "gemv_int8: K must be a positive multiple of 16");
  RH_REQUIRE(ldw >= K && ldw % 16 == 0 && ldw < (1 << 21),
             "gemv_int8: ldw must be >= K, < 2^21 and a multiple of 16");
  RH_REQUIRE(w8 != nullptr && scale != nullptr && x != nullptr, "gemv_int8: missing pointer");
  RH_REQUIRE((reinterpret_cast<uintptr_t>(w8) | reinterpret_cast<uintptr_t>(x)) % 16 == 0,
             "gemv_int8: W8 and x must be 16-byte aligned");
  return 0;
}

int check_rope(const float* inv_freq, const int* pos, const int* seq, const int* table_off, const int* tables,
               void* kpool, void* vpool, int heads, int kv_heads, int head_dim, int block_size) {
  RH_REQUIRE(inv_freq && pos && seq && table_off && tables && kpool && vpool, "qkv epilogue: missing pointer");
  RH_REQUIRE(heads > 0 && kv_heads > 0 && heads % kv_heads == 0, "qkv epilogue: bad head counts");
  RH_REQUIRE(head_dim > 0 && head_dim % 16 == 0, "qkv epilogue: head_dim must be a multiple of 16");
  RH_REQUIRE(block_size > 0, "qkv epilogue: bad block size");
  return 0;
}

// act = SiLU(gate) * up of the int8 gate/up product of RMSNorm(x), 1-8 tokens: the fused
// whole-line kernel with both prologue and SiLU epilogue (16 weight rows = 8 outputs per
// workgroup). With >= 256 workgroups it runs 8 waves of 2 steps, the K split of
// gemv_int8_m8_kernel, so the bytes equal rh_rmsnorm followed by rh_gemv_int8_gate_up_silu.
template <bool F16_SCALE>
int launch_m8_rmsnorm_silu(const int8_t* w8, int64_t ldw, const void* scale, const float* x, const float* norm_w,
                           float eps, half_t* act, int T, int K, int I, hipStream_t s) {
  const size_t staged = static_cast<size_t>(T) * (K + 8) * sizeof(half_t);
  RH_REQUIRE(staged <= kFusedLdsBytes, "gemv_int8: T * (K + 8) fp16 activations exceed the fused path's LDS");
  const int tiles = (I + 7) / 8, N = 2 * I;
  float* out = reinterpret_cast<float*>(act);
  if (tiles < 256) {
    RH_TRY_LAUNCH(hipLaunchKernelGGL((gemv_int8_m8_fused_kernel<16, 1, false, F16_SCALE, kRmsNorm, kSilu>), dim3(tiles),
                                     dim3(16 * kWave), staged, s, w8, ldw, scale, x, norm_w, eps, out, T, K, N, 0.0f,
                                     RopeArgs{}));
  } else {
    RH_TRY_LAUNCH(hipLaunchKernelGGL((gemv_int8_m8_fused_kernel<8, 2, false, F16_SCALE, kRmsNorm, kSilu>), dim3(tiles),
                                     dim3(8 * kWave), staged, s, w8, ldw, scale, x, norm_w, eps, out, T, K, N, 0.0f,
                                     RopeArgs{}));
  }
  return 0;
}

template <int PRO, int EPI>
int int8_fused(const int8_t* w8, int64_t ldw, const void* scale, int scale_is_f16, const void* xin,
               const float* norm_w, float eps, float* y, int T, int K, int N, float beta, void* stream,
               const RopeArgs& ra = RopeArgs{}) {
  if (int rc = check_int8_fused(w8, ldw, scale, xin, T, K, N, PRO == kPlain ? 2 * kMaxTokens : kMaxTokens)) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return scale_is_f16 ? launch_fused<true, PRO, EPI>(w8, ldw, scale, xin, norm_w, eps, y, T, K, N, beta, s, ra)
                      : launch_fused<false, PRO, EPI>(w8, ldw, scale, xin, norm_w, eps, y, T, K, N, beta, s, ra);
}

}  // namespace
}  // namespace relay_hip

using namespace relay_hip;

extern "C" int rh_gemv_int8_rmsnorm(const int8_t* w8, int64_t ldw, const void* scale, int scale_is_f16, const float* x,
                                    const float* norm_w, float eps, float* y, int T, int K, int N, float beta,
                                    void* stream) {
  RH_REQUIRE(norm_w != nullptr && reinterpret_cast<uintptr_t>(norm_w) % 16 == 0,
             "gemv_int8_rmsnorm: norm weights missing or not 16-byte aligned");
  return int8_fused<kRmsNorm, kStore>(w8, ldw, scale, scale_is_f16, x, norm_w, eps, y, T, K, N, beta, stream);
}

extern "C" int rh_gemv_int8_silu(const int8_t* w8, int64_t ldw, const void* scale, int scale_is_f16, const float* gu,
                                 float* y, int T, int K, int N, float beta, void* stream) {
  return int8_fused<kSiluMul, kStore>(w8, ldw, scale, scale_is_f16, gu, nullptr, 0.0f, y, T, K, N, beta, stream);
}

extern "C" int rh_gemv_int8_qkv(const int8_t* w8, int64_t ldw, const void* scale, int scale_is_f16, const void* x,
                                float* qkv, int T, int K, const float* bias, const float* inv_freq, const int* pos,
                                const int* seq, const int* table_off, const int* tables, void* kpool, void* vpool,
                                void* q_out, float q_scale, int heads, int kv_heads, int head_dim, int block_size,
                                void* stream) {
  if (int rc = check_rope(inv_freq, pos, seq, table_off, tables, kpool, vpool, heads, kv_heads, head_dim, block_size))
    return rc;
  RopeArgs ra{bias, inv_freq, pos, seq, table_off, tables, static_cast<half_t*>(kpool), static_cast<half_t*>(vpool),
              static_cast<half_t*>(q_out), q_scale, heads, kv_heads, head_dim, block_size};
  const int N = (heads + 2 * kv_heads) * head_dim;
  return int8_fused<kPlain, kRope>(w8, ldw, scale, scale_is_f16, x, nullptr, 0.0f, qkv, T, K, N, 0.0f, stream, ra);
}

extern "C" int rh_gemv_int8_rmsnorm_qkv(const int8_t* w8, int64_t ldw, const void* scale, int scale_is_f16,
                                        const float* x, const float* norm_w, float eps, float* qkv, int T, int K,
                                        const float* bias, const float* inv_freq, const int* pos, const int* seq,
                                        const int* table_off, const int* tables, void* kpool, void* vpool,
                                        void* q_out, float q_scale, int heads, int kv_heads, int head_dim,
                                        int block_size, void* stream) {
  RH_REQUIRE(norm_w != nullptr && reinterpret_cast<uintptr_t>(norm_w) % 16 == 0,
             "gemv_int8_rmsnorm_qkv: norm weights missing or not 16-byte aligned");
  if (int rc = check_rope(inv_freq, pos, seq, table_off, tables, kpool, vpool, heads, kv_heads, head_dim, block_size))
    return rc;
  RopeArgs ra{bias, inv_freq, pos, seq, table_off, tables, static_cast<half_t*>(kpool), static_cast<half_t*>(vpool),
              static_cast<half_t*>(q_out), q_scale, heads, kv_heads, head_dim, block_size};
  const int N = (heads + 2 * kv_heads) * head_dim;
  return int8_fused<kRmsNorm, kRope>(w8, ldw, scale, scale_is_f16, x, norm_w, eps, qkv, T, K, N, 0.0f, stream, ra);
}

extern "C" int rh_gemv_int8_max_tokens(void) { return kMaxInt8Tokens; }

extern "C" int64_t rh_gemv_int8_row_stride(int K) {
  if (K <= 0) return -1;
  const int64_t k = (static_cast<int64_t>(K) + 15) / 16 * 16;
  return k % 2048 == 0 ? k + 256 : k;
}

extern "C" int rh_gemv_int8(const int8_t* w8, int64_t ldw, const void* scale, int scale_is_f16, const void* x,
                            float* y, int T, int K, int N, float beta, void* stream) {
  RH_REQUIRE(T >= 1 && T <= kMaxInt8Tokens, "gemv_int8: T must be in 1..64");
  RH_REQUIRE(K > 0 && N > 0 && K % 16 == 0, "gemv_int8: K must be a positive multiple of 16");
  RH_REQUIRE(ldw >= K && ldw % 16 == 0 && ldw < (1 << 21),
             "gemv_int8: ldw must be >= K, < 2^21 and a multiple of 16");
  RH_REQUIRE((reinterpret_cast<uintptr_t>(w8) | reinterpret_cast<uintptr_t>(x)) % 16 == 0,
             "gemv_int8: W8 and x must be 16-byte aligned");
  RH_REQUIRE(w8 != nullptr && scale != nullptr && x != nullptr && y != nullptr, "gemv_int8: missing pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const half_t* xh = static_cast<const half_t*>(x);
  return scale_is_f16 ? launch<true>(w8, ldw, scale, xh, y, T, K, N, beta, s)
                      : launch<false>(w8, ldw, scale, xh, y, T, K, N, beta, s);
}

extern "C" int rh_gemv_int8_gate_up_silu(const int8_t* w8, int64_t ldw, const void* scale, int scale_is_f16,
                                         const void* x, void* act, int T, int K, int I, void* stream) {
  RH_REQUIRE(T >= 1 && T <= 16, "gemv_int8_gate_up_silu: T must be in 1..16");
  RH_REQUIRE(K > 0 && I > 0 && K % 16 == 0, "gemv_int8_gate_up_silu: K must be a positive multiple of 16");
  RH_REQUIRE(ldw >= K && ldw % 16 == 0 && ldw < (1 << 21),
             "gemv_int8_gate_up_silu: ldw must be >= K, < 2^21 and a multiple of 16");
  RH_REQUIRE((reinterpret_cast<uintptr_t>(w8) | reinterpret_cast<uintptr_t>(x)) % 16 == 0,
             "gemv_int8_gate_up_silu: W8 and x must be 16-byte aligned");
  RH_REQUIRE(w8 != nullptr && scale != nullptr && x != nullptr && act != nullptr, "gemv_int8_gate_up_silu: missing pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const half_t* xh = static_cast<const half_t*>(x);
  half_t* a = static_cast<half_t*>(act);
  if (T > 8) {  // two 8-token column blocks of the whole-line kernel, SiLU in its epilogue
    float* out = reinterpret_cast<float*>(act);
    return scale_is_f16 ? launch_whole_line<false, true, kPlain, kSilu>(w8, ldw, scale, x, nullptr, 0.0f, out, T, K,
                                                                        2 * I, 0.0f, s, RopeArgs{})
                        : launch_whole_line<false, false, kPlain, kSilu>(w8, ldw, scale, x, nullptr, 0.0f, out, T, K,
                                                                         2 * I, 0.0f, s, RopeArgs{});
  }
  return scale_is_f16 ? launch_m8_silu<true>(w8, ldw, scale, xh, a, T, K, I, s)
                      : launch_m8_silu<false>(w8, ldw, scale, xh, a, T, K, I, s);
}

extern "C" int rh_gemv_f16_gate_up_silu(const void* w16, int64_t ldw, const void* x, void* act, int T, int K, int I,
                                        void* stream) {
  RH_REQUIRE(T >= 1 && T <= 32, "gemv_f16_gate_up_silu: T must be in 1..32");
  RH_REQUIRE(K > 0 && I > 0 && K % 16 == 0, "gemv_f16_gate_up_silu: K must be a positive multiple of 16");
  RH_REQUIRE(ldw >= K && ldw % 8 == 0, "gemv_f16_gate_up_silu: ldw must be >= K and a multiple of 8");
  RH_REQUIRE(w16 != nullptr && x != nullptr && act != nullptr, "gemv_f16_gate_up_silu: missing pointer");
  RH_REQUIRE((reinterpret_cast<uintptr_t>(w16) | reinterpret_cast<uintptr_t>(x)) % 16 == 0,
             "gemv_f16_gate_up_silu: W16 and x must be 16-byte aligned");
  return launch_whole_line<true, false, kPlain, kSilu>(w16, ldw, nullptr, x, nullptr, 0.0f, static_cast<float*>(act), T,
                                                       K, 2 * I, 0.0f, static_cast<hipStream_t>(stream), RopeArgs{});
}

extern "C" int rh_gemv_int8_rmsnorm_gate_up_silu(const int8_t* w8, int64_t ldw, const void* scale, int scale_is_f16,
                                                 const float* x, const float* norm_w, float eps, void* act, int T,
                                                 int K, int I, void* stream) {
  RH_REQUIRE(T >= 1 && T <= 8, "gemv_int8_rmsnorm_gate_up_silu: T must be in 1..8");
  RH_REQUIRE(K > 0 && I > 0 && K % 16 == 0, "gemv_int8_rmsnorm_gate_up_silu: K must be a positive multiple of 16");
  RH_REQUIRE(ldw >= K && ldw % 16 == 0 && ldw < (1 << 21),
             "gemv_int8_rmsnorm_gate_up_silu: ldw must be >= K, < 2^21 and a multiple of 16");
  RH_REQUIRE(w8 != nullptr && scale != nullptr && x != nullptr && norm_w != nullptr && act != nullptr,
             "gemv_int8_rmsnorm_gate_up_silu: missing pointer");
  RH_REQUIRE((reinterpret_cast<uintptr_t>(w8) | reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(norm_w)) %
                     16 == 0,
             "gemv_int8_rmsnorm_gate_up_silu: W8, x and the norm weights must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  half_t* a = static_cast<half_t*>(act);
  return scale_is_f16 ? launch_m8_rmsnorm_silu<true>(w8, ldw, scale, x, norm_w, eps, a, T, K, I, s)
                      : launch_m8_rmsnorm_silu<false>(w8, ldw, scale, x, norm_w, eps, a, T, K, I, s);
}

extern "C" int rh_gemv_f16_max_tokens(void) { return 2 * kMaxTokens; }

namespace relay_hip {
namespace {

// fp16 weights at one token on the vector ALU: lane (rg =
// lane / 8, kl = lane % 8) reads the 8 halves W16[r0 + rg, k + 8 kl .. +8), so 8 lanes read
// 128 contiguous bytes of a row per load instruction, 8 rows per workgroup; v_dot2_f32_f16
// accumulates in fp32, lane shuffles sum a row's k-lanes and LDS the WAVES waves (which split
// K in runs of 64) in a fixed order.
template <int WAVES, int DEPTH>
__global__ __launch_bounds__(WAVES * kWave) void gemv_f16_t1_kernel(const half_t* __restrict__ wt, int64_t ldw,
                                                                    const half_t* __restrict__ x, float* y, int K,
                                                                    int N, float beta) {
  __shared__ float red[WAVES][8];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int rg = lane >> 3, kl = lane & 7;
  const int r0 = blockIdx.x * 8;
  const int nsteps = (K + 63) / 64;
  const int per = (nsteps + WAVES - 1) / WAVES;
  const int s0 = w * per, s1 = min(nsteps, s0 + per);
  const bool writer = threadIdx.x < 8 && r0 + static_cast<int>(threadIdx.x) < N;
  const float yold = writer && beta != 0.0f ? y[r0 + threadIdx.x] : 0.0f;  // before the weight stream
  const half_t* wr = wt + static_cast<int64_t>(min(r0 + rg, N - 1)) * ldw + 8 * kl;
  const half8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
  float acc = 0.0f;
  for (int st = s0; st < s1; st += DEPTH) {
    half8 a[DEPTH], xa[DEPTH];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      const int k = (st + d) * 64 + 8 * kl;
      const bool live = st + d < s1 && k < K;
      a[d] = live ? *reinterpret_cast<const half8*>(wr + (st + d) * 64) : zero;
      xa[d] = live ? *reinterpret_cast<const half8*>(x + k) : zero;
    }
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
#pragma unroll
      for (int e = 0; e < 8; e += 2)
        acc = __builtin_amdgcn_fdot2(half2_t{a[d][e], a[d][e + 1]}, half2_t{xa[d][e], xa[d][e + 1]}, acc, false);
  }
  acc += __shfl_xor(acc, 1);
  acc += __shfl_xor(acc, 2);
  acc += __shfl_xor(acc, 4);
  if (kl == 0) red[w][rg] = acc;
  __syncthreads();
  if (writer) {
    float v = 0.0f;
#pragma unroll
    for (int ww = 0; ww < WAVES; ++ww) v += red[ww][threadIdx.x];
    y[r0 + threadIdx.x] = v + (beta != 0.0f ? beta * yold : 0.0f);
  }
}

// fp16 weights at 2-8 tokens on the matrix cores with whole-line row loads (the layout of
// gemv_int8_m8_kernel): the 16 A rows of v_mfma_f32_16x16x32_f16 are 8 W rows x the two 32-k
// halves of a 64-k step, its 16 B columns 8 tokens x the same halves. Lane (c, g) loads the 8
// halves W16[r0 + c / 2, k + 32 (c % 2) + 8 g ..+8) straight into its A operand, so one load
// instruction covers 8 rows x 128 contiguous bytes, and token c / 2's activations at the same
// k into its B operand (zero past T). The C blocks whose row half matches the column half
// hold the sums; a lane shuffle adds the halves and LDS the WAVES waves in a fixed order.
template <int WAVES, int DEPTH>
__global__ __launch_bounds__(WAVES * kWave) void gemv_f16_m8_kernel(const half_t* __restrict__ wt, int64_t ldw,
                                                                    const half_t* __restrict__ x, float* y, int T,
                                                                    int K, int N, float beta) {
  __shared__ float red[WAVES][8][8];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int r = c >> 1, h = c & 1;
  const int r0 = blockIdx.x * 8;
  const int nsteps = (K + 63) / 64;
  const int per = (nsteps + WAVES - 1) / WAVES;
  const int s0 = w * per, s1 = min(nsteps, s0 + per);
  const int wt_ = threadIdx.x >> 3, wn = r0 + (threadIdx.x & 7);
  const bool writer = threadIdx.x < 8 * T && wn < N;
  const float yold = writer && beta != 0.0f ? y[static_cast<int64_t>(wt_) * N + wn] : 0.0f;  // before the weights
  const half_t* wr = wt + static_cast<int64_t>(min(r0 + r, N - 1)) * ldw + 32 * h + 8 * g;
  const bool tok = r < T;
  const half_t* xr = x + static_cast<int64_t>(tok ? r : 0) * K + 32 * h + 8 * g;
  const half8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
  float4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int st = s0; st < s1; st += DEPTH) {
    half8 a[DEPTH], b[DEPTH];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      const int k = (st + d) * 64 + 32 * h + 8 * g;
      const bool live = st + d < s1 && k < K;
      a[d] = live ? load_half8(wr + (st + d) * 64) : zero;
      b[d] = live && tok ? load_half8(xr + (st + d) * 64) : zero;
    }
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) acc = mfma16x16x32(a[d], b[d], acc);
  }
  // Lane (column 2t + h, g) holds C rows 4g + q = (W row 2g + q / 2, half q % 2).
  const float m0 = h ? acc[1] : acc[0], m1 = h ? acc[3] : acc[2];
  const float v0 = m0 + __shfl_xor(m0, 1), v1 = m1 + __shfl_xor(m1, 1);
  if (h == 0 && tok) {
    red[w][r][2 * g] = v0;
    red[w][r][2 * g + 1] = v1;
  }
  __syncthreads();
  if (writer) {
    float v = 0.0f;
#pragma unroll
    for (int ww = 0; ww < WAVES; ++ww) v += red[ww][wt_][threadIdx.x & 7];
    y[static_cast<int64_t>(wt_) * N + wn] = v + (beta != 0.0f ? beta * yold : 0.0f);
  }
}

// Plain fp16 products at 1-8 tokens (one token: below 2 Mi weights) take gemv_f16_m8_kernel: 8 waves of 4 steps, 4 waves of 8
// below 256 workgroups. Measured (us, 16-row tile -> this, T = 2 / 4 / 8): TinyLlama 2048 x
// 2048 5.8 / 6.0 / 6.2 -> 3.9 / 4.1 / 3.8, 2048 -> 11264 14.3 / 14.8 / 14.7 -> 9.2 / 9.4 /
// 10.6, 5632 -> 2048 9.8 / 10.1 / 11.2 -> 6.3 / 6.3 / 6.6; 4096 -> 14336 24.2 / 25.8 / 28.6
// -> 20.9 / 20.8 / 23.3; SmolLM2 1536 -> 576 4.5 / 4.6 / 4.9 -> 3.9 / 4.1 / 4.0, 576 -> 960
// level (~4.0, latency). One token too below gemv_f16_t1_kernel's range (SmolLM2-135M fp16
// decode step 0.816 -> 0.800 ms; on the t1 kernel's matrices the two were level).
bool f16_m8_takes(int T) { return T >= 1 && T <= 8; }

int launch_f16_m8(const half_t* wt, int64_t ldw, const half_t* x, float* y, int T, int K, int N, float beta,
                  hipStream_t s) {
  const int groups = (N + 7) / 8;
  if (groups < 256)
    RH_TRY_LAUNCH(hipLaunchKernelGGL((gemv_f16_m8_kernel<4, 8>), dim3(groups), dim3(4 * kWave), 0, s, wt, ldw, x, y, T,
                                     K, N, beta));
  else
    RH_TRY_LAUNCH(hipLaunchKernelGGL((gemv_f16_m8_kernel<8, 4>), dim3(groups), dim3(8 * kWave), 0, s, wt, ldw, x, y, T,
                                     K, N, beta));
  return 0;
}

// Whether a plain one-token product takes gemv_f16_t1_kernel: from 2 Mi weights (4 MB) up,
// where it measured faster than the MFMA tile (us: TinyLlama 2048 x 2048 5.7 -> 4.2, 2048 ->
// 11264 13.9 -> 9.0, 2048 -> 32000 27.3 -> 21.6, SmolLM2's 576 -> 49152 head 17.7 -> 10.4,
// 4096 x 4096 8.8 -> 7.4, 4096 -> 14336 23.7 -> 20.9); below, both take ~4 us of latency.
// 8 waves of 4 steps, 4 waves where K <= 1024.
bool f16_t1_takes(int T, int K, int N) { return T == 1 && static_cast<int64_t>(N) * K >= (int64_t{1} << 21); }

int launch_f16_t1(const half_t* wt, int64_t ldw, const half_t* x, float* y, int K, int N, float beta, hipStream_t s) {
  const int groups = (N + 7) / 8;
  if (K <= 1024)
    RH_TRY_LAUNCH(hipLaunchKernelGGL((gemv_f16_t1_kernel<4, 4>), dim3(groups), dim3(4 * kWave), 0, s, wt, ldw, x, y, K,
                                     N, beta));
  else
    RH_TRY_LAUNCH(hipLaunchKernelGGL((gemv_f16_t1_kernel<8, 4>), dim3(groups), dim3(8 * kWave), 0, s, wt, ldw, x, y, K,
                                     N, beta));
  return 0;
}

}  // namespace
}  // namespace relay_hip

template <int PRO, int EPI = kStore>
static int gemv_f16_launch(const void* w16, int64_t ldw, const void* x, const float* norm_w, float eps, float* y,
                           int T, int K, int N, float beta, void* stream, const RopeArgs& ra = RopeArgs{},
                           int ksplit = 1, const SplitArgs& sp = SplitArgs{}) {
  RH_REQUIRE(T >= 1 && T <= 2 * kMaxTokens, "gemv_f16: T must be in 1..32");
  RH_REQUIRE(K > 0 && N > 0 && K % 16 == 0, "gemv_f16: K must be a positive multiple of 16");
  RH_REQUIRE(ldw >= K && ldw % 8 == 0, "gemv_f16: ldw must be >= K and a multiple of 8");
  RH_REQUIRE((reinterpret_cast<uintptr_t>(w16) | reinterpret_cast<uintptr_t>(x)) % 16 == 0,
             "gemv_f16: W16 and x must be 16-byte aligned");
  const size_t staged = PRO == kPlain ? 0 : static_cast<size_t>(T) * (K + 8) * sizeof(half_t);
  RH_REQUIRE(staged <= kFusedLdsBytes, "gemv_f16: T * (K + 8) fp16 activations exceed the fused path's LDS");
  RH_REQUIRE(w16 != nullptr && x != nullptr && y != nullptr, "gemv_f16: missing pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const half_t* wt = static_cast<const half_t*>(w16);
  const int tiles = (N + 15) / 16;
  // 16 waves while the grid is below one workgroup per CU and each has >= 16 chunks of K.
  const bool wide = tiles * ksplit < 256 && (K + kChunk - 1) / kChunk / ksplit >= 16;
#define RH_GEMV_F16(W, NBLK)                                                                                    \
  RH_TRY_LAUNCH(hipLaunchKernelGGL((gemv_f16_kernel<W, NBLK, PRO, EPI>), dim3(tiles, ksplit), dim3(W * kWave),     \
                                   PRO == kPlain ? 0 : std::max<size_t>(staged, W * NBLK * kWave * 4 * sizeof(float)), s, wt, \
                                   ldw, x, norm_w, eps, y, T, K, N, beta, ra, sp))
  if (PRO == kPlain && EPI == kStore && ksplit == 1 && f16_t1_takes(T, K, N))
    return launch_f16_t1(wt, ldw, static_cast<const half_t*>(x), y, K, N, beta, s);
  if (PRO == kPlain && EPI == kStore && ksplit == 1 && f16_m8_takes(T))
    return launch_f16_m8(wt, ldw, static_cast<const half_t*>(x), y, T, K, N, beta, s);
  if (PRO == kPlain && EPI == kStore && ksplit == 1 && T >= 9)
    return launch_whole_line<true, false, kPlain, kStore>(wt, ldw, nullptr, x, nullptr, 0.0f, y, T, K, N, beta, s, ra);
  if constexpr (PRO != kPlain || EPI != kStore) {
    // A producer or the qkv epilogue at 1-16 tokens: the whole-line fused kernel.
    if (ksplit == 1 && T <= 32)
      return launch_whole_line<true, false, PRO, EPI>(wt, ldw, nullptr, x, norm_w, eps, y, T, K, N, beta, s, ra);
  }
  if (T <= kMaxTokens) {
    if (wide) {
      RH_GEMV_F16(16, 1);
    } else {
      RH_GEMV_F16(8, 1);
    }
  } else if (wide) {
    RH_GEMV_F16(16, 2);
  } else {
    RH_GEMV_F16(8, 2);
  }
#undef RH_GEMV_F16
  return 0;
}

extern "C" int rh_gemv_f16(const void* w16, int64_t ldw, const void* x, float* y, int T, int K, int N, float beta,
                           void* stream) {
  return gemv_f16_launch<kPlain>(w16, ldw, x, nullptr, 0.0f, y, T, K, N, beta, stream);
}

extern "C" int rh_gemv_f16_split_plan(int T, int K, int N) {
  if (T < 1 || K <= 0 || N <= 0) return -1;
  // Measured on MI355X (T = 1-32): the merge costs ~3 us (stores, counter, loads), so only
  // a long K on few row tiles gains (N = 2048, K = 5632, T = 32: 18.5 -> 14.4 us); ranges of
  // K on wider grids, or more than two, were slower everywhere.
  // Up to 16 tokens the whole-line kernel (8-row workgroups on such matrices) is faster
  // unsplit (5632 -> 2048 at T = 16: 8.8 us).
  const int tiles = (N + 15) / 16, nchunks = (K + kChunk - 1) / kChunk;
  return T > 16 && tiles <= 128 && nchunks >= 64 ? 2 : 1;
}

extern "C" int rh_gemv_f16_splitk(const void* w16, int64_t ldw, const void* x, float* y, int T, int K, int N,
                                  float beta, int ksplit, float* workspace, int* counters, void* stream) {
  RH_REQUIRE(ksplit >= 1 && ksplit <= kMaxSplit, "gemv_f16_splitk: ksplit must be in 1..8");
  RH_REQUIRE(ksplit <= (K + kChunk - 1) / kChunk, "gemv_f16_splitk: more K ranges than 64-wide chunks of K");
  RH_REQUIRE(ksplit == 1 || (workspace != nullptr && counters != nullptr),
             "gemv_f16_splitk: ksplit > 1 needs a workspace and counters");
  return gemv_f16_launch<kPlain>(w16, ldw, x, nullptr, 0.0f, y, T, K, N, beta, stream, RopeArgs{}, ksplit,
                                 SplitArgs{workspace, counters});
}

extern "C" int rh_gemv_f16_rmsnorm(const void* w16, int64_t ldw, const float* x, const float* norm_w, float eps,
                                   float* y, int T, int K, int N, float beta, void* stream) {
  RH_REQUIRE(norm_w != nullptr && reinterpret_cast<uintptr_t>(norm_w) % 16 == 0,
             "gemv_f16_rmsnorm: norm weights missing or not 16-byte aligned");
  return gemv_f16_launch<kRmsNorm>(w16, ldw, x, norm_w, eps, y, T, K, N, beta, stream);
}

extern "C" int rh_gemv_f16_silu(const void* w16, int64_t ldw, const float* gu, float* y, int T, int K, int N,
                                float beta, void* stream) {
  return gemv_f16_launch<kSiluMul>(w16, ldw, gu, nullptr, 0.0f, y, T, K, N, beta, stream);
}

extern "C" int rh_gemv_f16_qkv(const void* w16, int64_t ldw, const void* x, float* qkv, int T, int K,
                               const float* bias, const float* inv_freq, const int* pos, const int* seq,
                               const int* table_off, const int* tables, void* kpool, void* vpool, void* q_out,
                               float q_scale, int heads, int kv_heads, int head_dim, int block_size, void* stream) {
  RH_REQUIRE(inv_freq && pos && seq && table_off && tables && kpool && vpool, "gemv_f16_qkv: missing pointer");
  RH_REQUIRE(heads > 0 && kv_heads > 0 && heads % kv_heads == 0, "gemv_f16_qkv: bad head counts");
  RH_REQUIRE(head_dim > 0 && head_dim % 16 == 0, "gemv_f16_qkv: head_dim must be a multiple of 16");
  RH_REQUIRE(block_size > 0, "gemv_f16_qkv: bad block size");
  RopeArgs ra{bias, inv_freq, pos, seq, table_off, tables, static_cast<half_t*>(kpool), static_cast<half_t*>(vpool),
              static_cast<half_t*>(q_out), q_scale, heads, kv_heads, head_dim, block_size};
  const int N = (heads + 2 * kv_heads) * head_dim;
  return gemv_f16_launch<kPlain, kRope>(w16, ldw, x, nullptr, 0.0f, qkv, T, K, N, 0.0f, stream, ra);
}

extern "C" int rh_gemv_f16_rmsnorm_qkv(const void* w16, int64_t ldw, const float* x, const float* norm_w, float eps,
                                       float* qkv, int T, int K, const float* bias, const float* inv_freq,
                                       const int* pos, const int* seq, const int* table_off, const int* tables,
                                       void* kpool, void* vpool, void* q_out, float q_scale, int heads, int kv_heads,
                                       int head_dim, int block_size, void* stream) {
  RH_REQUIRE(norm_w != nullptr && inv_freq && pos && seq && table_off && tables && kpool && vpool,
             "gemv_f16_rmsnorm_qkv: missing pointer");
  RH_REQUIRE(reinterpret_cast<uintptr_t>(norm_w) % 16 == 0, "gemv_f16_rmsnorm_qkv: norm weights not 16-byte aligned");
  RH_REQUIRE(heads > 0 && kv_heads > 0 && heads % kv_heads == 0, "gemv_f16_rmsnorm_qkv: bad head counts");
  RH_REQUIRE(head_dim > 0 && head_dim % 16 == 0, "gemv_f16_rmsnorm_qkv: head_dim must be a multiple of 16");
  RH_REQUIRE(block_size > 0, "gemv_f16_rmsnorm_qkv: bad block size");
  RopeArgs ra{bias, inv_freq, pos, seq, table_off, tables, static_cast<half_t*>(kpool), static_cast<half_t*>(vpool),
              static_cast<half_t*>(q_out), q_scale, heads, kv_heads, head_dim, block_size};
  const int N = (heads + 2 * kv_heads) * head_dim;
  return gemv_f16_launch<kRmsNorm, kRope>(w16, ldw, x, norm_w, eps, qkv, T, K, N, 0.0f, stream, ra);
}

extern "C" int rh_gemv_f16_fused_fits(int T, int K) {
  return T >= 1 && T <= 2 * kMaxTokens && K > 0 &&
         static_cast<size_t>(T) * (K + 8) * sizeof(half_t) <= kFusedLdsBytes;
}
