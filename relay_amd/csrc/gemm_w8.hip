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

#include <algorithm>

namespace relay_hip {
namespace {

// int8 x 8 -> fp16 x 8, exact, in 10 instructions: each byte b ^ 0x80 (= b + 128 as an
// unsigned byte) is placed under a 0x64 high byte by v_perm_b32, which gives the fp16
// 1024 + b + 128, and 1152 is then subtracted (a packed fp16 add; exact).
__device__ __forceinline__ half8 int8x8_to_half8_w8(uint32_t lo, uint32_t hi) {
  const uint32_t x0 = lo ^ 0x80808080u, x1 = hi ^ 0x80808080u;
  const uint4v u = {__builtin_amdgcn_perm(0x64646464u, x0, 0x04010400u), __builtin_amdgcn_perm(0x64646464u, x0, 0x04030402u),
                    __builtin_amdgcn_perm(0x64646464u, x1, 0x04010400u), __builtin_amdgcn_perm(0x64646464u, x1, 0x04030402u)};
  const half8 bias = {1152, 1152, 1152, 1152, 1152, 1152, 1152, 1152};
  return __builtin_bit_cast(half8, u) - bias;
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

// ---- the large-batch tile (T above 64: prefill chunks, mixed batches) -------------------
//
// 4 waves; wave w owns rows 32 AN w .. +32 AN of the workgroup's 128 AN rows and all of its
// 32 BT tokens (AN x BT accumulators of v_mfma_f32_32x32x16_f16). Per 64-k step:
//   - W: lane (c, h) of a wave reads the 32 bytes W8[row c of block a, k0 + 32 h .. +32) as
//     two 16-byte buffer loads straight into registers, two steps ahead (two named register
//     sets for even and odd steps); in k-slice q its A operand holds k = k0 + 32 h + 8 q + j
//     in slot 8 h + j, converted from int8 just before use;
//   - x: the workgroup's 32 BT x 64 activation tile is loaded one step ahead and staged in
//     LDS (double-buffered, rows padded by 16 bytes: conflict-free 16-byte reads); lane (c, h)
//     reads x[t, k0 + 32 h + 8 q .. +8) as the matching B operand of token t = 32 b + c;
//   - the LDS reads and A conversions of k-slice q + 1 are issued before the MFMAs of slice q.
// Every load is unconditional (steps past the range re-read the last one, rows past N read
// row N - 1, tokens past T read row T - 1; none of those columns or rows is stored), so the
// compiler's wait counts stay exact. Workgroup L runs on XCD L % 8; each XCD takes a
// contiguous range of tiles with the token tile fastest, so the workgroups that share a W
// slice share an L2. K may be cut into ksn ranges (blockIdx-derived kz), written raw to a
// workspace and added in range order by w8_split_merge_kernel.
//
// Measured on MI355X, Llama-3-8B shapes at T = 560 (us; dequantize + rocBLAS in brackets,
// the fp16 library GEMM on fp16 weights in braces): 6144 x 4096 56.9 [~75] {42-46},
// 4096 x 4096 44.0 [~60] {29-40}, 28672 x 4096 166.9 (the 2 x 3 tile) [~200] {128-135},
// 4096 x 14336 103.4 [~125] {87-105}. A copy of the kernel without the global loads in the
// loop runs the 28672 x 4096 product in 103 us, so the remaining gap to the MFMA rate is the
// memory pipeline (W and x loads cost ~40 and ~20 us there). Tried and slower: one wave per
// SIMD with 4 x 4 or 4 x 3 blocks per wave, 4 x 2 blocks, token-major tile order, per-slice
// scheduling barriers.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t w8_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7fffffff, 0x00020000);
}

template <int AN, int BT, int WPE>
__global__ __launch_bounds__(256, WPE) void w8_tile_kernel(const int8_t* __restrict__ w8, int64_t ldw,
                                                           const float* __restrict__ scale,
                                                           const half_t* __restrict__ x, float* y, int T, int K, int N,
                                                           float beta, float* ws, int n_row, int n_tok, int ksn,
                                                           int vec_out) {
  constexpr int KS = 64, XR = KS + 8, RB = 128 * AN, TB = 32 * BT;
  __shared__ __attribute__((aligned(16))) half_t xs[2][TB * XR];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, c = lane & 31, h = lane >> 5;
  const int total = n_row * n_tok * ksn, L = blockIdx.x;
  const int per = total / 8, rem = total % 8, xcd = L % 8;
  const int idx = xcd * per + min(xcd, rem) + L / 8;
  const int tok = idx % n_tok, rk = idx / n_tok, kz = rk % ksn, row = rk / ksn;
  const int n0 = row * RB, t0 = tok * TB;
  const int nall = K / KS, sbeg = kz * nall / ksn, nsteps = (kz + 1) * nall / ksn - sbeg;

  const __amdgpu_buffer_rsrc_t wrs = w8_rsrc(w8 + static_cast<int64_t>(n0) * ldw + static_cast<int64_t>(sbeg) * KS);
  const __amdgpu_buffer_rsrc_t xrs = w8_rsrc(x + static_cast<int64_t>(sbeg) * KS);
  int woff[AN];
#pragma unroll
  for (int a = 0; a < AN; ++a)
    woff[a] = (min(n0 + 32 * (AN * w + a) + c, N - 1) - n0) * static_cast<int>(ldw) + 32 * h;
  int xoff[BT];  // activation piece j of this thread: token e / 8, k piece e % 8, e = tid + 256 j
#pragma unroll
  for (int j = 0; j < BT; ++j) {
    const int e = tid + 256 * j, t = min(t0 + e / 8, T - 1);
    xoff[j] = (t * K + 8 * (e % 8)) * 2;
  }
  uint4v wa[AN][2], wb[AN][2];
  uint4v xr[BT];
  auto load_w = [&](uint4v (&wr)[AN][2], int s) {
    const int so = min(s, nsteps - 1) * KS;
#pragma unroll
    for (int a = 0; a < AN; ++a)
#pragma unroll
      for (int v = 0; v < 2; ++v) wr[a][v] = __builtin_amdgcn_raw_buffer_load_b128(wrs, woff[a] + 16 * v, so, 0);
  };
  auto load_x = [&](int s) {
    const int so = min(s, nsteps - 1) * KS * 2;
#pragma unroll
    for (int j = 0; j < BT; ++j) xr[j] = __builtin_amdgcn_raw_buffer_load_b128(xrs, xoff[j], so, 0);
  };
  auto stage = [&](int buf) {
#pragma unroll
    for (int j = 0; j < BT; ++j) {
      const int e = tid + 256 * j;
      *reinterpret_cast<uint4v*>(&xs[buf][(e / 8) * XR + 8 * (e % 8)]) = xr[j];
    }
  };
  float16v acc[AN][BT];
#pragma unroll
  for (int a = 0; a < AN; ++a)
#pragma unroll
    for (int b = 0; b < BT; ++b)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[a][b][i] = 0.0f;

  auto compute = [&](const uint4v (&wr)[AN][2], int buf) {
    const half_t* xb = &xs[buf][c * XR + 32 * h];
    half8 bq[2][BT], av[2][AN];
#pragma unroll
    for (int b = 0; b < BT; ++b) bq[0][b] = *reinterpret_cast<const half8*>(xb + 32 * b * XR);
#pragma unroll
    for (int a = 0; a < AN; ++a) av[0][a] = int8x8_to_half8_w8(wr[a][0][0], wr[a][0][1]);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int cu = q & 1, nx = cu ^ 1;
      if (q < 3) {
#pragma unroll
        for (int b = 0; b < BT; ++b) bq[nx][b] = *reinterpret_cast<const half8*>(xb + 32 * b * XR + 8 * (q + 1));
#pragma unroll
        for (int a = 0; a < AN; ++a)
          av[nx][a] = int8x8_to_half8_w8(wr[a][(q + 1) >> 1][2 * ((q + 1) & 1)], wr[a][(q + 1) >> 1][2 * ((q + 1) & 1) + 1]);
      }
#pragma unroll
      for (int a = 0; a < AN; ++a)
#pragma unroll
        for (int b = 0; b < BT; ++b) acc[a][b] = mfma32x32x16(av[cu][a], bq[cu][b], acc[a][b]);
    }
  };
  // Step s issues x(s + 1), computes s, then issues W(s + 2) into the set s just used.
  // The loop has one back edge and no exit in its body (an exit there made the compiler
  // keep two copies of the accumulators); an odd last step runs after it.
  load_x(0);
  load_w(wa, 0);
  load_w(wb, 1);
  stage(0);
  __syncthreads();
  int s = 0;
  for (; s + 1 < nsteps; s += 2) {
    load_x(s + 1);
    compute(wa, 0);
    load_w(wa, s + 2);
    stage(1);
    __syncthreads();
    load_x(s + 2);
    compute(wb, 1);
    load_w(wb, s + 3);
    stage(0);
    __syncthreads();
  }
  if (s < nsteps) compute(wa, 0);

  // Register 4 q + r of block (a, b) in lane (c, h): row 32 (AN w + a) + 8 q + 4 h + r,
  // token 32 b + c.
#pragma unroll
  for (int b = 0; b < BT; ++b) {
    const int t = t0 + 32 * b + c;
    if (t >= T) continue;
#pragma unroll
    for (int a = 0; a < AN; ++a)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + 32 * (AN * w + a) + 8 * q + 4 * h;
        if (n >= N) continue;
        float4v v = {acc[a][b][4 * q], acc[a][b][4 * q + 1], acc[a][b][4 * q + 2], acc[a][b][4 * q + 3]};
        if (ksn > 1) {  // the host requires N % 4 == 0 here
          *reinterpret_cast<float4v*>(ws + (static_cast<int64_t>(kz) * T + t) * N + n) = v;
        } else if (vec_out && n + 3 < N) {
          const float4v sc = {scale[n], scale[n + 1], scale[n + 2], scale[n + 3]};
          float* yp = y + static_cast<int64_t>(t) * N + n;
          v = v * sc;
          if (beta != 0.0f) v += beta * *reinterpret_cast<const float4v*>(yp);
          *reinterpret_cast<float4v*>(yp) = v;
        } else {
          float* yp = y + static_cast<int64_t>(t) * N;
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n + r < N) {
              const float o = v[r] * scale[n + r];
              yp[n + r] = o + (beta != 0.0f ? beta * yp[n + r] : 0.0f);
            }
        }
      }
  }
}

// Tiles: 128 rows x 128 tokens (3 waves per SIMD fit), or 256 x 96 (2 per SIMD) when the
// grid already has >= 768 of the smaller tiles (28672 x 4096 at T = 560: 183 -> 167 us).
struct W8TilePlan {
  bool big;
  int ksplit;
};

W8TilePlan w8_tile_plan(int T, int K, int N) {
  const int small = ((N + 127) / 128) * ((T + 127) / 128);
  if (small >= 768) return {true, 1};
  // K ranges until the grid has >= 480 workgroups (about two per CU), at most 8 and each
  // at least 4 steps of 64 k (measured at Llama-3-8B and TinyLlama shapes, T = 128-560).
  int ks = small >= 384 ? 1 : std::min(8, (480 + small - 1) / small);
  while (ks > 1 && (K / 64) / ks < 4) --ks;
  if (N % 4) ks = 1;
  return {false, ks};
}

template <int AN, int BT, int WPE>
int launch_w8_tile(const int8_t* w8, int64_t ldw, const float* scale, const half_t* x, float* y, int T, int K, int N,
                   float beta, hipStream_t s, int ksplit, float* ws) {
  const int n_row = (N + 128 * AN - 1) / (128 * AN), n_tok = (T + 32 * BT - 1) / (32 * BT);
  const int64_t total = static_cast<int64_t>(n_row) * n_tok * ksplit;
  RH_REQUIRE(total < (int64_t(1) << 31), "gemm_w8: grid too large");
  const int vec_out = N % 4 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0;
  RH_TRY_LAUNCH(hipLaunchKernelGGL((w8_tile_kernel<AN, BT, WPE>), dim3(static_cast<unsigned>(total)), dim3(256), 0, s,
                                   w8, ldw, scale, x, y, T, K, N, beta, ws, n_row, n_tok, ksplit, vec_out));
  if (ksplit > 1) {
    const int64_t quads = static_cast<int64_t>(T) * N / 4;
    RH_TRY_LAUNCH(hipLaunchKernelGGL(w8_split_merge_kernel, dim3(static_cast<unsigned>((quads + 255) / 256)), dim3(256), 0,
                                     s, ws, ksplit, T, N, scale, y, beta));
  }
  return 0;
}

// The tile for 17-64 tokens: 128 rows x 64 tokens, 4 waves of 32 rows (the 128-token tile
// leaves most MFMA columns idle there and gives 4x fewer row tiles per token).
constexpr int kSkinnyRows = 128, kSkinnyTokens = 64;

}  // namespace
}  // namespace relay_hip

using namespace relay_hip;


static int gemm_w8_checks(const int8_t* w8, int64_t ldw, const void* x, int T, int K, int N) {
  RH_REQUIRE(T > 0 && N > 0 && K > 0 && K % 64 == 0, "gemm_w8: K must be a positive multiple of 64");
  RH_REQUIRE(ldw >= K && ldw % 16 == 0, "gemm_w8: ldw must be >= K and a multiple of 16");
  RH_REQUIRE((reinterpret_cast<uintptr_t>(w8) | reinterpret_cast<uintptr_t>(x)) % 16 == 0,
             "gemm_w8: W8 and x must be 16-byte aligned");
  RH_REQUIRE(static_cast<int64_t>(T) * K < (int64_t(1) << 30) && 256 * ldw < (int64_t(1) << 31),
             "gemm_w8: T * K or the row stride too large for 32-bit buffer offsets");
  return 0;
}

extern "C" int rh_gemm_w8(const int8_t* w8, int64_t ldw, const float* scale, const void* x, float* y, int T, int K,
                          int N, float beta, void* stream) {
  if (T == 0) return 0;
  if (int rc = gemm_w8_checks(w8, ldw, x, T, K, N)) return rc;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const half_t* xh = static_cast<const half_t*>(x);
  if (w8_tile_plan(T, K, N).big) return launch_w8_tile<2, 3, 2>(w8, ldw, scale, xh, y, T, K, N, beta, st, 1, nullptr);
  return launch_w8_tile<1, 4, 3>(w8, ldw, scale, xh, y, T, K, N, beta, st, 1, nullptr);
}

extern "C" int rh_gemm_w8_plan(int T, int K, int N) {
  if (T < 1 || K <= 0 || K % 64 || N <= 0) return -1;
  return w8_tile_plan(T, K, N).ksplit;
}

extern "C" int rh_gemm_w8_split(const int8_t* w8, int64_t ldw, const float* scale, const void* x, float* y, int T,
                                int K, int N, float beta, int ksplit, float* workspace, void* stream) {
  if (T == 0) return 0;
  if (int rc = gemm_w8_checks(w8, ldw, x, T, K, N)) return rc;
  RH_REQUIRE(ksplit >= 1 && ksplit <= kMaxW8Split && ksplit <= K / 64,
             "gemm_w8_split: ksplit must be in 1..8 and at most the number of 64-k steps");
  RH_REQUIRE(ksplit == 1 || workspace, "gemm_w8_split: ksplit > 1 needs a workspace");
  RH_REQUIRE(ksplit == 1 || N % 4 == 0, "gemm_w8_split: ksplit > 1 needs N a multiple of 4");
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const half_t* xh = static_cast<const half_t*>(x);
  if (ksplit == 1 && w8_tile_plan(T, K, N).big)
    return launch_w8_tile<2, 3, 2>(w8, ldw, scale, xh, y, T, K, N, beta, st, 1, nullptr);
  return launch_w8_tile<1, 4, 3>(w8, ldw, scale, xh, y, T, K, N, beta, st, ksplit, workspace);
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
