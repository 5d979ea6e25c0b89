// Weight-only int8 GEMM for batches above the GEMV's token limit, on the matrix cores:
//
//   y[t, n] = scale[n] * sum_k W8[n, k] * x[t, k]  (+ beta * y[t, n])
//
// relay runs this case as a dequantization of the whole matrix to an fp16 scratch followed
// by a dense GEMM (cuda_backend.cu:710-722): the weights cross HBM three times (int8 read,
// fp16 write, fp16 read). Here the int8 bytes are read once and converted in registers to
// the fp16 A operands of v_mfma_f32_32x32x16_f16 (exact: int8 values are integers that
// fp16 holds, and int8 x fp16 products are exact in the fp32 accumulator); the per-row
// scale multiplies the finished sums, as in the int8 GEMV, so both int8 paths compute the
// same function.
//
// Workgroup: 4 waves, a 64 (rows of W) x 128 (tokens) tile of y. Wave (wn, wt) owns rows
// n0 + 32 wn .. +32 and tokens t0 + 64 wt .. +64 (two 32x32 accumulators). Per 64-k step:
//   - lane (c, h) of a wave loads the 32 bytes W8[n0 + 32 wn + c, k0 + 32 h .. +32) straight
//     into registers (one step ahead) and splits them into four 8-byte A operands; in
//     MFMA step q its k slots 8h + j hold k = k0 + 32h + 8q + j;
//   - the workgroup stages the 128 x 64 fp16 activation tile in LDS (double-buffered, rows
//     padded by 16 bytes); lane (c, h) reads x[t, k0 + 32h + 8q .. +8) as the matching B
//     operand of token t = t0 + 64 wt + 32 cb + c.
// One barrier per step: step s reads buffer s & 1 and fills buffer (s + 1) & 1, which every
// wave finished reading before the previous barrier.
//
// Measured on MI355X at Llama-3-8B shapes: 430-470 TFLOP/s where the grid has >= 1000
// workgroups (N = 28672, T = 560), 280-400 on the 32-48-tile grids of N = 4096-6144; it wins
// while the weights dominate (T up to a few hundred), and dequantize + library GEMM wins
// once the product is compute-bound. 128x128 tiles, 128-k steps and prefetching 2-4 steps
// ahead through more register sets were all slower (the registers cut occupancy). The
// template keeps the tile shape and prefetch depth as parameters.
//
// rh_gemm_w8_skinny (17-64 tokens) instantiates it with a 128-row x 64-token tile and
// 128-k steps, and cuts K into ranges over blockIdx.z so that narrow matrices still cover
// the GPU (Llama-3-8B down projection at T = 48: 47.2 us with the GEMV, 28.6 us with 8
// ranges); a second launch adds the ranges' partial sums in order.
#include "../../include/relay_hip.h"
#include "common.h"

namespace relay_hip {
namespace {

__device__ __forceinline__ half8 int8x8_to_half8_w8(uint32_t lo, uint32_t hi) {
  // bytes b -> halves with bits 0x6400 | (b ^ 0x80) = 1024 + b + 128, minus 1152.
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

// WN x WT waves; each wave AN 32-row blocks x BT 32-token blocks.
template <int WN, int WT, int AN, int BT, int KS>
struct Tile {
  static constexpr int kXRow = KS + 8;  // halves per staged activation row
  static constexpr int kPR = KS / 8;    // 16-byte pieces per activation row
  static constexpr int kWV = KS / 32;   // 16-byte W loads per lane and row block
  static constexpr int kThreads = 64 * WN * WT;
  static constexpr int kRows = 32 * AN * WN;
  static constexpr int kToks = 32 * BT * WT;
  static constexpr int kPieces = kToks * kPR / kThreads;  // 16-byte activation pieces per thread
};

// Split K (gridDim.z > 1): each workgroup takes a range of K steps and writes its raw sums
// to ws [ksn][T][N]; w8_split_merge_kernel then adds the ranges in order and applies the
// scale and beta (a second launch: a merge inside this kernel by the last workgroup to
// arrive needed registers that cut the main loop's occupancy from 4 waves per SIMD to 1).
struct W8Split {
  float* ws;
};

template <int WN, int WT, int AN, int BT, int KS, int PF>
__global__ __launch_bounds__(64 * WN * WT) void gemm_w8_kernel(const int8_t* __restrict__ w8, int64_t ldw,
                                                              const float* __restrict__ scale,
                                                              const half_t* __restrict__ x, float* y, int T, int K,
                                                              int N, float beta, W8Split sp) {
  using TL = Tile<WN, WT, AN, BT, KS>;
  constexpr int kXRow = TL::kXRow, kPR = TL::kPR, kWV = TL::kWV;
  __shared__ __attribute__((aligned(16))) half_t xs[2][TL::kToks * kXRow];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wn = w % WN, wt = w / WN, c = lane & 31, h = lane >> 5;
  const int n0 = blockIdx.x * TL::kRows, t0 = blockIdx.y * TL::kToks;
  const int8_t* wp[AN];
#pragma unroll
  for (int a = 0; a < AN; ++a)
    wp[a] = w8 + static_cast<int64_t>(min(n0 + 32 * (AN * wn + a) + c, N - 1)) * ldw + (KS / 2) * h;
  const int ksn = gridDim.z, kz = blockIdx.z;
  const int nall = K / KS, sbeg = kz * nall / ksn, nsteps = (kz + 1) * nall / ksn - sbeg;

  // Activation loader: thread tid moves 16-byte pieces e = tid + kThreads j of the tile
  // (token e / kPR, k piece e % kPR). Tokens past T re-read row T - 1: a token's column of
  // the accumulators depends only on its own row, and those columns are never stored, so
  // every load is unconditional (no branches around the loads).
  const half_t* xp[TL::kPieces];
#pragma unroll
  for (int j = 0; j < TL::kPieces; ++j) {
    const int e = tid + TL::kThreads * j, t = min(t0 + e / kPR, T - 1);
    xp[j] = x + static_cast<int64_t>(t) * K + 8 * (e % kPR);
  }
  // PF register sets: stage s is loaded into set s % PF, PF steps before it is used.
  uint4v wr[PF][AN][kWV];
  half8 xr[PF][TL::kPieces];
  auto load = [&](int s, int u) {
    const int k0 = (sbeg + s) * KS;
#pragma unroll
    for (int a = 0; a < AN; ++a)
#pragma unroll
      for (int v = 0; v < kWV; ++v) wr[u][a][v] = *reinterpret_cast<const uint4v*>(wp[a] + k0 + 16 * v);
#pragma unroll
    for (int j = 0; j < TL::kPieces; ++j) xr[u][j] = load_half8(xp[j] + k0);
  };
  auto stage = [&](int buf, int u) {
#pragma unroll
    for (int j = 0; j < TL::kPieces; ++j) {
      const int e = tid + TL::kThreads * j;
      *reinterpret_cast<half8*>(&xs[buf][(e / kPR) * kXRow + 8 * (e % kPR)]) = xr[u][j];
    }
  };

  float16v acc[AN][BT];
#pragma unroll
  for (int a = 0; a < AN; ++a)
#pragma unroll
    for (int b = 0; b < BT; ++b)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[a][b][i] = 0.0f;

#pragma unroll
  for (int u = 0; u < PF; ++u)
    if (u < nsteps) load(u, u);
  stage(0, 0);
  __syncthreads();
  for (int s0 = 0; s0 < nsteps; s0 += PF) {
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      const int s = s0 + u;
      if (s >= nsteps) break;
      half8 av[AN][KS / 16];
#pragma unroll
      for (int a = 0; a < AN; ++a)
#pragma unroll
        for (int q = 0; q < KS / 16; ++q) {
          const uint4v& wq = wr[u][a][q >> 1];
          av[a][q] = int8x8_to_half8_w8(wq[2 * (q & 1)], wq[2 * (q & 1) + 1]);
        }
      if (s + PF < nsteps) load(s + PF, u);
      const half_t* xb = &xs[s & 1][(32 * BT * wt + c) * kXRow + (KS / 2) * h];
#pragma unroll
      for (int q = 0; q < KS / 16; ++q) {
        half8 bq[BT];
#pragma unroll
        for (int b = 0; b < BT; ++b) bq[b] = *reinterpret_cast<const half8*>(xb + 32 * b * kXRow + 8 * q);
#pragma unroll
        for (int a = 0; a < AN; ++a)
#pragma unroll
          for (int b = 0; b < BT; ++b) acc[a][b] = mfma32x32x16(av[a][q], bq[b], acc[a][b]);
      }
      if (s + 1 < nsteps) stage((s + 1) & 1, (u + 1) % PF);
      __syncthreads();
    }
  }

  // Accumulator register i of lane (c, h) holds row 8 (i / 4) + 4 h + i % 4 of its 32-row
  // block, for token column c.
  if (ksn > 1) {
#pragma unroll
    for (int b = 0; b < BT; ++b) {
      const int t = t0 + 32 * (BT * wt + b) + c;
      if (t >= T) continue;
      float* part = sp.ws + (static_cast<int64_t>(kz) * T + t) * N;
#pragma unroll
      for (int a = 0; a < AN; ++a)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int n = n0 + 32 * (AN * wn + a) + 8 * q + 4 * h + r;
            if (n < N) part[n] = acc[a][b][4 * q + r];
          }
    }
    return;
  }
#pragma unroll
  for (int b = 0; b < BT; ++b) {
    const int t = t0 + 32 * (BT * wt + b) + c;
    if (t >= T) continue;
    float* yr = y + static_cast<int64_t>(t) * N;
#pragma unroll
    for (int a = 0; a < AN; ++a)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int n = n0 + 32 * (AN * wn + a) + 8 * q + 4 * h + r;
          if (n >= N) continue;
          const float v = acc[a][b][4 * q + r] * scale[n];
          yr[n] = v + (beta != 0.0f ? beta * yr[n] : 0.0f);
        }
  }
}

// y[t, n] = scale[n] * sum_z ws[z][t][n] (+ beta y), the ranges added in order; one thread
// per 4 consecutive n of a token row, all ksn loads in flight.
constexpr int kMaxW8Split = 8;
__global__ __launch_bounds__(256) void w8_split_merge_kernel(const float* __restrict__ ws, int ksn, int T, int N,
                                                             const float* __restrict__ scale, float* y, float beta) {
  const int64_t i4 = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (i4 >= static_cast<int64_t>(T) * N) return;
  const int64_t plane = static_cast<int64_t>(T) * N;
  const int n = static_cast<int>(i4 % N);
  float p[kMaxW8Split][4];
#pragma unroll
  for (int z = 0; z < kMaxW8Split; ++z)
#pragma unroll
    for (int e = 0; e < 4; ++e) p[z][e] = z < ksn ? ws[z * plane + i4 + e] : 0.0f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float v = 0.0f;
#pragma unroll
    for (int z = 0; z < kMaxW8Split; ++z)
      if (z < ksn) v += p[z][e];
    const float o = v * scale[n + e];
    y[i4 + e] = o + (beta != 0.0f ? beta * y[i4 + e] : 0.0f);
  }
}

template <int WN, int WT, int AN, int BT, int KS, int PF>
int launch_w8(const int8_t* w8, int64_t ldw, const float* scale, const half_t* x, float* y, int T, int K, int N,
              float beta, hipStream_t s, int ksplit = 1, W8Split sp = W8Split{}) {
  using TL = Tile<WN, WT, AN, BT, KS>;
  const dim3 grid((N + TL::kRows - 1) / TL::kRows, (T + TL::kToks - 1) / TL::kToks, ksplit);
  RH_REQUIRE(grid.y <= 65535, "gemm_w8: T too large");
  RH_TRY_LAUNCH(hipLaunchKernelGGL((gemm_w8_kernel<WN, WT, AN, BT, KS, PF>), grid, dim3(TL::kThreads), 0, s, w8, ldw, scale,
                                   x, y, T, K, N, beta, sp));
  if (ksplit > 1) {
    const int64_t quads = static_cast<int64_t>(T) * N / 4;
    RH_TRY_LAUNCH(hipLaunchKernelGGL(w8_split_merge_kernel, dim3(static_cast<unsigned>((quads + 255) / 256)), dim3(256), 0,
                                     s, sp.ws, ksplit, T, N, scale, y, beta));
  }
  return 0;
}

// The tile for 17-64 tokens: 128 rows x 64 tokens, 4 waves of 32 rows (the 128-token tile
// leaves most MFMA columns idle there and gives 4x fewer row tiles per token).
constexpr int kSkinnyRows = 128, kSkinnyTokens = 64;

}  // namespace
}  // namespace relay_hip

using namespace relay_hip;


extern "C" int rh_gemm_w8(const int8_t* w8, int64_t ldw, const float* scale, const void* x, float* y, int T, int K,
                          int N, float beta, void* stream) {
  if (T == 0) return 0;
  RH_REQUIRE(T > 0 && N > 0 && K > 0 && K % 64 == 0, "gemm_w8: K must be a positive multiple of 64");
  RH_REQUIRE(ldw >= K && ldw % 16 == 0, "gemm_w8: ldw must be >= K and a multiple of 16");
  RH_REQUIRE((reinterpret_cast<uintptr_t>(w8) | reinterpret_cast<uintptr_t>(x)) % 16 == 0,
             "gemm_w8: W8 and x must be 16-byte aligned");
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const half_t* xh = static_cast<const half_t*>(x);
  return launch_w8<2, 2, 1, 2, 64, 1>(w8, ldw, scale, xh, y, T, K, N, beta, st);
}

// k per step of the skinny tile: 128 when K allows (measured 10-15% faster than 64 at
// 32-48 tokens; deeper register prefetch of the weights gained nothing).
static int skinny_step(int K) { return K % 128 == 0 ? 128 : 64; }

extern "C" int rh_gemm_w8_split_plan(int T, int K, int N) {
  if (T < 1 || T > kSkinnyTokens || K <= 0 || K % 64 || N <= 0) return -1;
  // The fewest K ranges that give >= 256 workgroups (one per CU), each range >= 8 steps.
  // Measured at Llama-3-8B shapes, T = 32-48: N = 4096, K = 14336 best with 8 ranges,
  // N = 28672, K = 4096 with 2; more ranges than that were slower.
  const int tiles = (N + kSkinnyRows - 1) / kSkinnyRows, steps = K / skinny_step(K);
  int ks = 1;
  while (tiles * ks < 256 && 2 * ks <= kMaxW8Split && steps / (2 * ks) >= 8) ks *= 2;
  return ks;
}

extern "C" int rh_gemm_w8_skinny(const int8_t* w8, int64_t ldw, const float* scale, const void* x, float* y, int T,
                                 int K, int N, float beta, int ksplit, float* workspace, void* stream) {
  if (T == 0) return 0;
  RH_REQUIRE(T > 0 && T <= kSkinnyTokens, "gemm_w8_skinny: T must be in 1..64");
  RH_REQUIRE(N > 0 && K > 0 && K % 64 == 0, "gemm_w8_skinny: K must be a positive multiple of 64");
  RH_REQUIRE(ldw >= K && ldw % 16 == 0, "gemm_w8_skinny: ldw must be >= K and a multiple of 16");
  RH_REQUIRE((reinterpret_cast<uintptr_t>(w8) | reinterpret_cast<uintptr_t>(x)) % 16 == 0,
             "gemm_w8_skinny: W8 and x must be 16-byte aligned");
  RH_REQUIRE(ksplit >= 1 && ksplit <= kMaxW8Split && ksplit <= K / skinny_step(K),
             "gemm_w8_skinny: ksplit must be in 1..8 and at most the number of k steps");
  RH_REQUIRE(ksplit == 1 || workspace, "gemm_w8_skinny: ksplit > 1 needs a workspace");
  RH_REQUIRE(ksplit == 1 || N % 4 == 0, "gemm_w8_skinny: ksplit > 1 needs N a multiple of 4");
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const half_t* xh = static_cast<const half_t*>(x);
  if (skinny_step(K) == 128)
    return launch_w8<4, 1, 1, 2, 128, 1>(w8, ldw, scale, xh, y, T, K, N, beta, st, ksplit, W8Split{workspace});
  return launch_w8<4, 1, 1, 2, 64, 1>(w8, ldw, scale, xh, y, T, K, N, beta, st, ksplit, W8Split{workspace});
}
