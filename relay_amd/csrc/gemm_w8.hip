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
// same function. One kernel template serves every batch size from 17 tokens up, with the
// tile chosen per range (w8_tile_kernel below); K may be cut into ranges that a second
// launch adds in order.
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
    const float o = mul_rounded(v, scale[n + e]);
    y[i4 + e] = o + (beta != 0.0f ? beta * y[i4 + e] : 0.0f);
  }
}

// ---- the tile kernel -------------------------------------------------------------------
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

// The tile's results: register 4 q + r of block (a, b) in lane (c, h) is row 32 (AN w + a) +
// 8 q + 4 h + r, token 32 b + c. ksn > 1: this K range's raw sums go to the workspace (the
// host requires N % 4 == 0 there) and w8_split_merge_kernel (or a consumer) adds the ranges
// in order. (A merge by the last workgroup of each tile to arrive, through coherent stores
// and loads and an arrival counter, measured 1.4-6x slower than the merge launch at T =
// 32-560: the partials are written through.)
template <int AN, int BT>
__device__ __forceinline__ void w8_write_out(const float16v (&acc)[AN][BT], int w, int c, int h, int n0, int t0, int kz,
                                             int T, int N, int ksn, float* ws, const float* __restrict__ scale, float* y,
                                             float beta, int vec_out) {
  auto store = [&](float4v v, int t, int n) {
    if (vec_out && n + 3 < N) {
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
          const float o = mul_rounded(v[r], scale[n + r]);
          yp[n + r] = o + (beta != 0.0f ? beta * yp[n + r] : 0.0f);
        }
    }
  };
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
        const float4v v = {acc[a][b][4 * q], acc[a][b][4 * q + 1], acc[a][b][4 * q + 2], acc[a][b][4 * q + 3]};
        if (ksn > 1)
          *reinterpret_cast<float4v*>(ws + (static_cast<int64_t>(kz) * T + t) * N + n) = v;
        else
          store(v, t, n);
      }
  }
}

// SILU (AN = 2, one K range): W is the fused [gate; up] matrix (N = 2 I rows) and the tile
// holds the 128 outputs a0 .. a0 + 127 (a0 = 128 x its row index): block 0 of wave w gate
// rows a0 + 32 w .. +32, block 1 the up rows I rows further, so every accumulator register
// of block 0 has its partner at the same place in block 1 and the epilogue writes act[t, a]
// = fp16(silu(g) * u) (fp16 [T, I]) instead of y -- the values of the plain product
// followed by silu_mul_vec_kernel.
template <int AN, int BT, int WPE, bool SILU = false>
__global__ __launch_bounds__(256, WPE) void w8_tile_kernel(const int8_t* __restrict__ w8, int64_t ldw,
                                                           const float* __restrict__ scale,
                                                           const half_t* __restrict__ x, float* y, int T, int K, int N,
                                                           float beta, float* ws, int n_row, int n_tok, int ksn,
                                                           int vec_out) {
  static_assert(!SILU || AN == 2, "the SiLU tile pairs gate and up blocks");
  constexpr int KS = 64, XR = KS + 8, RB = SILU ? 128 : 128 * AN, TB = 32 * BT;
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
  const int I = N / 2;  // SILU only
  int woff[AN];
#pragma unroll
  for (int a = 0; a < AN; ++a)
    woff[a] = SILU ? (min(n0 + 32 * w + c, I - 1) - n0 + a * I) * static_cast<int>(ldw) + 32 * h
                   : (min(n0 + 32 * (AN * w + a) + c, N - 1) - n0) * static_cast<int>(ldw) + 32 * h;
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
  if constexpr (AN * BT == 2 || AN * BT == 4) {
    // The 128 x 64 and 128 x 128 tiles: one back edge and no exit in the loop body (an exit
    // there made the compiler keep two copies of the accumulators); an odd last step runs
    // after it.
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
  } else {
    // The 128 x 32 and 256 x 96 tiles: pairs of steps, the second under a (uniform) test.
    // Measured against the form above, same process (us): 256 x 96 at 28672 x 4096, T = 560
    // 168.5 -> 160.7; 128 x 32 at T = 32, 4096 x 14336 in 8 ranges 24.8 -> 21.8, 2048 x 5632
    // in 8 ranges 12.3 -> 11.7, 11264 x 2048 in 2 ranges 15.2 -> 13.6. (On the 128 x 64 tile
    // this form was slower: 40.6 -> 51.2 at 4096 x 14336, T = 32, 4 ranges.)
    load_w(wa, 0);
    load_w(wb, 1);
    load_x(0);
    stage(0);
    __syncthreads();
    for (int s = 0; s < nsteps; s += 2) {
      load_x(s + 1);
      compute(wa, 0);
      load_w(wa, s + 2);
      stage(1);
      __syncthreads();
      if (s + 1 < nsteps) {
        load_x(s + 2);
        compute(wb, 1);
        load_w(wb, s + 3);
        stage(0);
      }
      __syncthreads();
    }
  }

  if constexpr (SILU) {
    half_t* act = reinterpret_cast<half_t*>(y);
#pragma unroll
    for (int b = 0; b < BT; ++b) {
      const int t = t0 + 32 * b + c;
      if (t >= T) continue;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int a = n0 + 32 * w + 8 * q + 4 * h;
        half_t o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int ar = min(a + r, I - 1);
          // the values w8_write_out's vector store gives y (sum x scale, rounded once)
          const float g = mul_rounded(acc[0][b][4 * q + r], scale[ar]);
          const float u = mul_rounded(acc[1][b][4 * q + r], scale[I + ar]);
          o[r] = f16_of_product(g / (1.0f + expf(-g)), u);
        }
        half_t* dst = act + static_cast<int64_t>(t) * I + a;
        if (vec_out && a + 3 < I) {
          *reinterpret_cast<half4*>(dst) = half4{o[0], o[1], o[2], o[3]};
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (a + r < I) dst[r] = o[r];
        }
      }
    }
  } else {
    w8_write_out<AN, BT>(acc, w, c, h, n0, t0, kz, T, N, ksn, ws, scale, y, beta, vec_out);
  }
}

// ---- the wide-step kernel ---------------------------------------------------------------
//
// 128 rows x 32 BT tokens, 4 waves (wave w: rows 32 w .. +32, all tokens), two workgroups per
// CU. Per 128-k step lane (c, h) reads the 64 contiguous bytes W8[row c, k0 + 64 h .. +64)
// (four 16-byte loads), and k-slice j (j = 0..7) takes slots 8 h .. 8 h + 7 from k0 + 64 h +
// 8 j on both operands, so every lane's bytes of a step are one half of a 128-byte line.
// W runs two steps ahead in two register sets, x two steps ahead in two register sets
// staged into a double-buffered LDS tile. Steps come in pairs with no branch inside; a
// step past the range (the second of an odd count) computes with a zero x tile, so its
// products add exact zeros. Measured against the 64-k tile kernel (us, in isolation; the
// kernel / its best K split at each point): Llama-3-8B at T = 560: 6144 x 4096 45.6 / 56.9,
// 4096 x 4096 37.8 (96-token tile) / 44.4, 4096 x 14336 100.2 / 107.3; at T = 512:
// TinyLlama 2560 x 2048 20.9 / 29.8, 11264 x 2048 42.2 / 58.7, 2048 x 5632 30.1 / 35.7.
template <int BT>
__global__ __launch_bounds__(256, 2) void w8_wide_kernel(const int8_t* __restrict__ w8, int64_t ldw,
                                                         const float* __restrict__ scale, const half_t* __restrict__ x,
                                                         float* y, int T, int K, int N, float beta, float* ws,
                                                         int n_row, int n_tok, int ksn, int vec_out) {
  constexpr int KS = 128, XR = KS + 8, TB = 32 * BT, NX = 2 * BT;  // NX 16-byte x pieces per thread
  __shared__ __attribute__((aligned(16))) half_t xs[2][TB * XR];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, c = lane & 31, h = lane >> 5;
  const int total = n_row * n_tok * ksn, L = blockIdx.x;
  const int per = total / 8, rem = total % 8, xcd = L % 8;
  const int idx = xcd * per + min(xcd, rem) + L / 8;
  const int tok = idx % n_tok, rk = idx / n_tok, kz = rk % ksn, row = rk / ksn;
  const int n0 = row * 128, t0 = tok * TB;
  const int nall = K / KS, sbeg = kz * nall / ksn, nsteps = (kz + 1) * nall / ksn - sbeg;

  const __amdgpu_buffer_rsrc_t wrs = w8_rsrc(w8 + static_cast<int64_t>(n0) * ldw + static_cast<int64_t>(sbeg) * KS);
  const __amdgpu_buffer_rsrc_t xrs = w8_rsrc(x + static_cast<int64_t>(sbeg) * KS);
  const int woff = (min(n0 + 32 * w + c, N - 1) - n0) * static_cast<int>(ldw) + 64 * h;
  int xoff[NX], xst[NX];  // piece j: token e / 16, k piece e % 16, e = tid + 256 j
#pragma unroll
  for (int j = 0; j < NX; ++j) {
    const int e = tid + 256 * j, r = e / 16, col = e % 16;
    xoff[j] = (min(t0 + r, T - 1) * K + 8 * col) * 2;
    xst[j] = r * XR + 8 * col;
  }
  uint4v wr[2][4], xr[2][NX];
  auto load_w = [&](int u, int s) {
    const int so = min(s, nsteps - 1) * KS;
#pragma unroll
    for (int v = 0; v < 4; ++v) wr[u][v] = __builtin_amdgcn_raw_buffer_load_b128(wrs, woff + 16 * v, so, 0);
  };
  auto load_x = [&](int u, int s) {
    const int so = min(s, nsteps - 1) * KS * 2;
#pragma unroll
    for (int j = 0; j < NX; ++j) xr[u][j] = __builtin_amdgcn_raw_buffer_load_b128(xrs, xoff[j], so, 0);
  };
  auto stage = [&](int u, bool live) {
#pragma unroll
    for (int j = 0; j < NX; ++j) {
      uint4v v = xr[u][j];
      if (!live) v = uint4v{0u, 0u, 0u, 0u};
      *reinterpret_cast<uint4v*>(&xs[u][xst[j]]) = v;
    }
  };
  float16v acc[1][BT];
#pragma unroll
  for (int b = 0; b < BT; ++b)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[0][b][i] = 0.0f;

  auto compute = [&](int u) {
    const half_t* xb = &xs[u][c * XR + 64 * h];
    half8 bq[2][BT], av[2];
#pragma unroll
    for (int b = 0; b < BT; ++b) bq[0][b] = *reinterpret_cast<const half8*>(xb + 32 * b * XR);
    av[0] = int8x8_to_half8_w8(wr[u][0][0], wr[u][0][1]);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int cu = j & 1, nx = cu ^ 1;
      if (j < 7) {
#pragma unroll
        for (int b = 0; b < BT; ++b) bq[nx][b] = *reinterpret_cast<const half8*>(xb + 32 * b * XR + 8 * (j + 1));
        av[nx] = int8x8_to_half8_w8(wr[u][(j + 1) >> 1][2 * ((j + 1) & 1)], wr[u][(j + 1) >> 1][2 * ((j + 1) & 1) + 1]);
      }
#pragma unroll
      for (int b = 0; b < BT; ++b) acc[0][b] = mfma32x32x16(av[cu], bq[cu][b], acc[0][b]);
    }
  };
  // Step s: issue x(s + 2) into x set s & 1 (staged already), compute s from LDS buffer
  // s & 1, issue W(s + 2) into W set s & 1, stage x(s + 1) into LDS buffer (s + 1) & 1.
  load_w(0, 0);
  load_x(0, 0);
  load_w(1, 1);
  load_x(1, 1);
  stage(0, true);
  __syncthreads();
  for (int s = 0; s < nsteps; s += 2) {
    load_x(0, s + 2);
    compute(0);
    load_w(0, s + 2);
    stage(1, s + 1 < nsteps);
    __syncthreads();
    load_x(1, s + 3);
    compute(1);
    load_w(1, s + 3);
    stage(0, s + 2 < nsteps);
    __syncthreads();
  }
  w8_write_out<1, BT>(acc, w, c, h, n0, t0, kz, T, N, ksn, ws, scale, y, beta, vec_out);
}

template <int BT>
int launch_w8_wide(const int8_t* w8, int64_t ldw, const float* scale, const half_t* x, float* y, int T, int K, int N,
                   float beta, hipStream_t s, int ksplit, float* ws) {
  // ksplit < 0: -ksplit ranges, partials only (no merge launch; a fused consumer merges).
  const bool merge = ksplit > 0;
  ksplit = merge ? ksplit : -ksplit;
  const int n_row = (N + 127) / 128, n_tok = (T + 32 * BT - 1) / (32 * BT);
  const int64_t total = static_cast<int64_t>(n_row) * n_tok * ksplit;
  RH_REQUIRE(total < (int64_t(1) << 31), "gemm_w8: grid too large");
  const int vec_out = N % 4 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0;
  RH_TRY_LAUNCH(hipLaunchKernelGGL((w8_wide_kernel<BT>), dim3(static_cast<unsigned>(total)), dim3(256), 0, s, w8, ldw,
                                   scale, x, y, T, K, N, beta, ws, n_row, n_tok, ksplit, vec_out));
  if (ksplit > 1 && merge) {
    const int64_t quads = static_cast<int64_t>(T) * N / 4;
    RH_TRY_LAUNCH(hipLaunchKernelGGL(w8_split_merge_kernel, dim3(static_cast<unsigned>((quads + 255) / 256)), dim3(256), 0,
                                     s, ws, ksplit, T, N, scale, y, beta));
  }
  return 0;
}

// Kernels and K splits above 64 tokens. kTile128 (w8_tile_kernel<1, 4, 3>) and kTileBig
// (<2, 3, 2>, 256 x 96) take any K that is a multiple of 64; the wide-step kernels
// (128 x 128 and 128 x 96 tiles) need K a multiple of 128 and at least one 128-k step per
// range.
enum W8Cfg { kTile128 = 0, kTileBig = 1, kWide128 = 2, kWide96 = 3 };
struct W8Plan {
  int cfg;
  int ksplit;
};

// The previous plan, kept for K not a multiple of 128: the 128 x 128 tile with K ranges
// until the grid has >= 480 workgroups (at most 8 ranges of >= 4 steps), or the 256 x 96
// tile when there are >= 768 of the smaller tiles.
W8Plan w8_tile_plan(int T, int K, int N) {
  const int small = ((N + 127) / 128) * ((T + 127) / 128);
  if (small >= 768) return {kTileBig, 1};
  int ks = small >= 384 ? 1 : std::min(8, (480 + small - 1) / small);
  while (ks > 1 && (K / 64) / ks < 4) --ks;
  if (N % 4) ks = 1;
  return {kTile128, ks};
}

// A timing model of one product, in microseconds, fitted to 1088 measured (kernel, split)
// pairs over eight Llama-3-8B and TinyLlama matrices at eight T from 128 to 560 (log-RMS
// error 5.6%).
// A workgroup's time is (128-k steps in its range + 1.83) x a per-tile factor (the
// 128 x 96 tile 0.85, 256 x 96 1.34 of the 128 x 128 one), nearly independent of how many
// tokens its tile holds; the grid runs as rounds of 256 workgroups (two share a CU, at the
// same total rate; one alone runs at 0.95 / 0.88 / 0.70 of it); a split adds its merge,
// 2.16 us + 1.53 us per million partial sums read and written. Choosing the minimum of the
// model picks a kernel within 1.3% of the measured best on average over those points
// (worst 11%), against 22% above it for the previous plan.
// With consumer_merge the partials are added by the product's consumer (rh_w8_merge_rmsnorm /
// rh_w8_merge_silu) in place of a launch it makes anyway: the split then costs only the
// reads of its extra ranges, 1.53 us per million partial sums.
double w8_model_us(int cfg, int T, int K, int N, int ks, bool consumer_merge = false) {
  const int rows = cfg == kTileBig ? 256 : 128, toks = cfg == kWide128 ? 128 : 96;
  const double factor = cfg == kWide128 ? 1.0 : cfg == kWide96 ? 0.8513 : 1.34;
  const double alone = cfg == kWide128 ? 0.8826 : cfg == kWide96 ? 0.9462 : 0.7039;
  const int64_t wgs = static_cast<int64_t>((N + rows - 1) / rows) * ((T + toks - 1) / toks) * ks;
  const double w = (K / 128.0 / ks + 1.8343) * factor;
  const int64_t rounds = (wgs + 255) / 256;
  double t = static_cast<double>(rounds / 2) * 2.0 * w + static_cast<double>(rounds % 2) * w / alone;
  if (ks > 1 && consumer_merge) return t + 1.5261e-6 * (ks - 1) * static_cast<double>(T) * N;
  if (ks > 1) t += 2.1571 + 1.5261e-6 * (ks + 1) * static_cast<double>(T) * N;
  return t;
}

int64_t w8_grid(int cfg, int T, int N) {
  const int rows = cfg == kTileBig ? 256 : 128, toks = cfg == kWide128 ? 128 : 96;
  return static_cast<int64_t>((N + rows - 1) / rows) * ((T + toks - 1) / toks);
}

bool w8_wide_fits(int K, int ks) { return K % 128 == 0 && ks <= K / 128; }

// The kernel for a given split: the model's choice among the kernels that take it.
int w8_cfg_for(int T, int K, int N, int ks) {
  if (T <= 64 || !w8_wide_fits(K, ks)) return ks == 1 && w8_tile_plan(T, K, N).cfg == kTileBig ? kTileBig : kTile128;
  int best = kWide128;
  double tb = w8_model_us(kWide128, T, K, N, ks);
  for (int cfg : {kWide96, kTileBig}) {
    if (cfg == kTileBig && ks != 1) continue;
    const double t = w8_model_us(cfg, T, K, N, ks);
    if (t < tb) tb = t, best = cfg;
  }
  return best;
}

// Kernel and split: the model's minimum over the wide-step kernels at 1-8 ranges of >= 2
// steps and the 256 x 96 tile unsplit.
W8Plan w8_plan(int T, int K, int N) {
  if (T <= 64 || K % 128) return w8_tile_plan(T, K, N);
  W8Plan best = {kTileBig, 1};
  double tb = w8_model_us(kTileBig, T, K, N, 1);
  for (int ks = 1; ks <= kMaxW8Split && (K / 128) / ks >= 2; ++ks) {
    if (ks > 1 && N % 4) break;
    for (int cfg : {kWide128, kWide96}) {
      const double t = w8_model_us(cfg, T, K, N, ks);
      if (t < tb) tb = t, best = {cfg, ks};
    }
  }
  return best;
}

template <int AN, int BT, int WPE>
int launch_w8_tile(const int8_t* w8, int64_t ldw, const float* scale, const half_t* x, float* y, int T, int K, int N,
                   float beta, hipStream_t s, int ksplit, float* ws) {
  // ksplit < 0: -ksplit ranges, partials only (no merge launch; a fused consumer merges).
  const bool merge = ksplit > 0;
  ksplit = merge ? ksplit : -ksplit;
  const int n_row = (N + 128 * AN - 1) / (128 * AN), n_tok = (T + 32 * BT - 1) / (32 * BT);
  const int64_t total = static_cast<int64_t>(n_row) * n_tok * ksplit;
  RH_REQUIRE(total < (int64_t(1) << 31), "gemm_w8: grid too large");
  const int vec_out = N % 4 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0;
  RH_TRY_LAUNCH(hipLaunchKernelGGL((w8_tile_kernel<AN, BT, WPE>), dim3(static_cast<unsigned>(total)), dim3(256), 0, s,
                                   w8, ldw, scale, x, y, T, K, N, beta, ws, n_row, n_tok, ksplit, vec_out));
  if (ksplit > 1 && merge) {
    const int64_t quads = static_cast<int64_t>(T) * N / 4;
    RH_TRY_LAUNCH(hipLaunchKernelGGL(w8_split_merge_kernel, dim3(static_cast<unsigned>((quads + 255) / 256)), dim3(256), 0,
                                     s, ws, ksplit, T, N, scale, y, beta));
  }
  return 0;
}

// act = SiLU(gate) * up of the fused [gate; up] product on the 256 x 96 tile, one K range.
int launch_w8_tile_silu(const int8_t* w8, int64_t ldw, const float* scale, const half_t* x, half_t* act, int T, int K,
                        int I, hipStream_t s) {
  const int n_row = (I + 127) / 128, n_tok = (T + 95) / 96;
  const int64_t total = static_cast<int64_t>(n_row) * n_tok;
  RH_REQUIRE(total < (int64_t(1) << 31), "gemm_w8: grid too large");
  const int vec_out = I % 4 == 0 && reinterpret_cast<uintptr_t>(act) % 8 == 0;
  RH_TRY_LAUNCH(hipLaunchKernelGGL((w8_tile_kernel<2, 3, 2, true>), dim3(static_cast<unsigned>(total)), dim3(256), 0, s,
                                   w8, ldw, scale, x, reinterpret_cast<float*>(act), T, K, 2 * I, 0.0f, nullptr, n_row,
                                   n_tok, 1, vec_out));
  return 0;
}

int launch_w8_cfg(int cfg, const int8_t* w8, int64_t ldw, const float* scale, const half_t* x, float* y, int T, int K,
                  int N, float beta, hipStream_t s, int ksplit, float* ws) {
  switch (cfg) {
    case kTileBig: return launch_w8_tile<2, 3, 2>(w8, ldw, scale, x, y, T, K, N, beta, s, ksplit, ws);
    case kWide128: return launch_w8_wide<4>(w8, ldw, scale, x, y, T, K, N, beta, s, ksplit, ws);
    case kWide96: return launch_w8_wide<3>(w8, ldw, scale, x, y, T, K, N, beta, s, ksplit, ws);
    default: return launch_w8_tile<1, 4, 3>(w8, ldw, scale, x, y, T, K, N, beta, s, ksplit, ws);
  }
}

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
  return launch_w8_cfg(w8_cfg_for(T, K, N, 1), w8, ldw, scale, xh, y, T, K, N, beta, st, 1, nullptr);
}

extern "C" int rh_gemm_w8_gate_up_silu(const int8_t* w8, int64_t ldw, const float* scale, const void* x, void* act,
                                       int T, int K, int I, void* stream) {
  if (T == 0) return 0;
  RH_REQUIRE(I > 0, "gemm_w8_gate_up_silu: I must be positive");
  RH_REQUIRE(w8 != nullptr && scale != nullptr && x != nullptr && act != nullptr,
             "gemm_w8_gate_up_silu: missing pointer");
  if (int rc = gemm_w8_checks(w8, ldw, x, T, K, 2 * I)) return rc;
  RH_REQUIRE((static_cast<int64_t>(I) + 256) * ldw < (int64_t(1) << 31),
             "gemm_w8_gate_up_silu: I * ldw too large for 32-bit buffer offsets");
  return launch_w8_tile_silu(w8, ldw, scale, static_cast<const half_t*>(x), static_cast<half_t*>(act), T, K, I,
                             static_cast<hipStream_t>(stream));
}

extern "C" int rh_gemm_w8_plan(int T, int K, int N) {
  if (T < 1 || K <= 0 || K % 64 || N <= 0) return -1;
  return w8_plan(T, K, N).ksplit;
}

// The split for a product whose consumer merges it. Where the plan runs the product unsplit
// on fewer than 256 workgroups, the model prices a lone round below what it measures on such
// grids (Llama-3-8B's o projection, 4096 x 4096 at T = 560: 30 us modelled, 38-44 measured),
// so there the K is split over the ranges the model prices lowest with the consumer's merge
// (the o projection takes 3 ranges on the 128 x 128 tile: Llama-3-8B int8 mixed step 21.23 ->
// 21.10 ms; the down projection's plan, 3 ranges, was already the best of 2-5).
int w8_partials_plan(int T, int K, int N) {
  const W8Plan p = w8_plan(T, K, N);
  if (T <= 64 || K % 128 || N % 4 || p.ksplit > 1 || w8_grid(p.cfg, T, N) >= 256) return p.ksplit;
  int best = 1;
  double tb = 0.0;
  for (int ks = 2; ks <= kMaxW8Split && (K / 128) / ks >= 2; ++ks) {
    for (int cfg : {kWide128, kWide96}) {
      const double t = w8_model_us(cfg, T, K, N, ks, true);
      if (best == 1 || t < tb) tb = t, best = ks;
    }
  }
  return best;
}

extern "C" int rh_gemm_w8_partials_plan(int T, int K, int N) {
  if (T < 1 || K <= 0 || K % 64 || N <= 0) return -1;
  return w8_partials_plan(T, K, N);
}

extern "C" int rh_gemm_w8_kernel(int T, int K, int N, int ksplit) {
  if (T < 1 || K <= 0 || K % 64 || N <= 0 || ksplit < 1 || ksplit > kMaxW8Split || ksplit > K / 64) return -1;
  return w8_cfg_for(T, K, N, ksplit);
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
  return launch_w8_cfg(w8_cfg_for(T, K, N, ksplit), w8, ldw, scale, xh, y, T, K, N, beta, st, ksplit, workspace);
}

extern "C" int rh_gemm_w8_partials(const int8_t* w8, int64_t ldw, const void* x, int T, int K, int N, int ksplit,
                                   float* workspace, void* stream) {
  if (T == 0) return 0;
  if (int rc = gemm_w8_checks(w8, ldw, x, T, K, N)) return rc;
  RH_REQUIRE(ksplit >= 2 && ksplit <= kMaxW8Split && ksplit <= K / 64 && workspace && N % 4 == 0,
             "gemm_w8_partials: ksplit in 2..8 (at most K / 64), a workspace and N a multiple of 4");
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const half_t* xh = static_cast<const half_t*>(x);
  // No scale is read: the partials are the raw sums. The tile is the one the merging entry
  // point takes for this T.
  if (T <= 64 && w8_wide_fits(K, ksplit))
    return T <= 32 ? launch_w8_wide<1>(w8, ldw, nullptr, xh, nullptr, T, K, N, 0.0f, st, -ksplit, workspace)
                   : launch_w8_wide<2>(w8, ldw, nullptr, xh, nullptr, T, K, N, 0.0f, st, -ksplit, workspace);
  if (T <= 32) return launch_w8_tile<1, 1, 4>(w8, ldw, nullptr, xh, nullptr, T, K, N, 0.0f, st, -ksplit, workspace);
  if (T <= 64) return launch_w8_tile<1, 2, 4>(w8, ldw, nullptr, xh, nullptr, T, K, N, 0.0f, st, -ksplit, workspace);
  return launch_w8_cfg(w8_cfg_for(T, K, N, ksplit), w8, ldw, nullptr, xh, nullptr, T, K, N, 0.0f, st, -ksplit, workspace);
}

// 17-64 tokens: the wide-step kernel with a 32-token tile (64 above 32 tokens) where K is
// a multiple of 128, else the 64-k tile kernel (128 rows x 32 or 64 tokens, four waves per
// SIMD, K cut until the row tiles x ranges reach 256 workgroups, at most 8 ranges of >= 4
// steps). The wide-step kernel, measured against the tile kernel at the tile kernel's plan
// (us, in isolation, merge launch included; T = 32 / 64): 28672 x 4096 31.2 / 38.1 against
// 35.8 / 45.6, 4096 x 14336 20.4 / 24.7 against 22.7 / 28.9, 6144 x 4096 14.7 / 17.9 against
// 17.5 / 22.0, 11264 x 2048 14.8 against 17.7, 2048 x 5632 13.2 / 15.6 against 13.5 / 16.2;
// TinyLlama int8 decode steps 1.676 -> 1.617 ms at b = 32, 1.587 -> 1.540 at 24, 1.464 ->
// 1.424 at 17. (Loading W four steps ahead in the tile kernel instead: 1-7% slower.)
// The tile kernel (us, in isolation, T = 32; the GEMV and a 128-row x 64-token tile in
// brackets): 28672 x 4096 32.8 [-, 34.0], 4096 x 14336 24.3 [-, 26.9], TinyLlama 2048 x
// 5632 12.3 [15.2, 14.9], 11264 x 2048 15.0 [15.7, 17.7]; on K <= 4096 matrices of <= 6144
// rows the GEMV stays ahead (4096 x 4096: 12.5 against 13.5).
constexpr int kSkinnyTokens = 64;

extern "C" int rh_gemm_w8_split_plan(int T, int K, int N) {
  if (T < 1 || T > kSkinnyTokens || K <= 0 || K % 64 || N <= 0) return -1;
  // (One range from 64 row tiles up, to save the merge launch, made the TinyLlama int8
  // 32 x 2048 decode step slower: 1.80 -> 1.91 ms.)
  const int tiles = (N + 127) / 128;
  if (K % 128 == 0) {
    // The wide-step kernel: as many ranges (of >= 2 steps) as keep the grid within one
    // workgroup per CU; one more round of a few workgroups costs more than the ranges save
    // (T = 32, 11264 x 2048: 2 ranges 14.8 us, 3 ranges 18.4).
    int ks = std::max(1, std::min(8, 256 / tiles));
    while (ks > 1 && (K / 128) / ks < 2) --ks;
    return N % 4 ? 1 : ks;
  }
  int ks = std::min(8, (256 + tiles - 1) / tiles);
  while (ks > 1 && (K / 64) / ks < 4) --ks;
  return N % 4 ? 1 : ks;
}

extern "C" int rh_gemm_w8_skinny(const int8_t* w8, int64_t ldw, const float* scale, const void* x, float* y, int T,
                                 int K, int N, float beta, int ksplit, float* workspace, void* stream) {
  if (T == 0) return 0;
  RH_REQUIRE(T > 0 && T <= kSkinnyTokens, "gemm_w8_skinny: T must be in 1..64");
  if (int rc = gemm_w8_checks(w8, ldw, x, T, K, N)) return rc;
  RH_REQUIRE(ksplit >= 1 && ksplit <= kMaxW8Split && ksplit <= K / 64,
             "gemm_w8_skinny: ksplit must be in 1..8 and at most the number of 64-k steps");
  RH_REQUIRE(ksplit == 1 || workspace, "gemm_w8_skinny: ksplit > 1 needs a workspace");
  RH_REQUIRE(ksplit == 1 || N % 4 == 0, "gemm_w8_skinny: ksplit > 1 needs N a multiple of 4");
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const half_t* xh = static_cast<const half_t*>(x);
  if (w8_wide_fits(K, ksplit))
    return T <= 32 ? launch_w8_wide<1>(w8, ldw, scale, xh, y, T, K, N, beta, st, ksplit, workspace)
                   : launch_w8_wide<2>(w8, ldw, scale, xh, y, T, K, N, beta, st, ksplit, workspace);
  if (T <= 32) return launch_w8_tile<1, 1, 4>(w8, ldw, scale, xh, y, T, K, N, beta, st, ksplit, workspace);
  return launch_w8_tile<1, 2, 4>(w8, ldw, scale, xh, y, T, K, N, beta, st, ksplit, workspace);
}
