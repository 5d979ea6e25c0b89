// Flash prefill attention over the paged KV cache for gfx950 (fp16 MFMA, fp32 softmax).
//
// Work unit: one workgroup per (tile of up to 128 consecutive query rows of one chunk,
// query head), four waves of 32 rows -- the role of relay's flash_prefill_kernel<D>
// (cuda_kernels.cuh:28-178), re-cut for 64-wide waves and 32x32 matrix cores. The
// workgroup walks the keys 0 .. (last row's position) 64 at a time; each 64-key tile of
// K and V is gathered through the block table into LDS once for the four waves.
//
// Per wave and 32-key sub-tile:
//   S^T[32 keys x 32 rows] = K[32 keys x D] * Q^T[D x 32 rows]         (D/16 MFMA 32x32x16)
//   online softmax per query row: lane = row, so the row max and sum are reductions over
//   the lane's own 16 registers plus one swap with lane l^32
//   O^T[D x 32 rows] += V^T[D x 32 keys] * P^T[32 keys x 32 rows]       (D/16 MFMA 32x32x16)
// The S^T accumulators are the P^T B operands as they stand (registers 0-7 and 8-15 are
// the two 16-key halves, in the same permuted key order the V^T A operand is read in),
// so P never goes through LDS. The 1/sqrt(D) scale and log2(e) fold into the exp2
// argument (one FMA per score). O^T is rescaled only when some row's maximum grew.
//
// LDS rows are XOR-swizzled in 16-byte chunks: K by key & 7 (the 32 keys of an A-operand
// read spread over all banks), V by bit 2 of the key (the two key groups of a transposed
// read land in different halves of the banks).
//
// Workgroups are ordered heaviest tile first, and when the head count is a multiple of 8
// each XCD (workgroup ids are dealt round-robin over the 8 XCDs) gets a contiguous
// range of heads, i.e. few KV heads, so its L2 holds the K/V it re-reads.
#include "../../include/relay_hip.h"
#include "common.h"

namespace relay_hip {
namespace {

constexpr int kRows = 128;      // query rows per workgroup
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * kWave;
constexpr int kKeyTile = 64;    // keys per LDS tile

struct PrefillArgs {
  const half_t* q;
  int64_t q_stride;
  const half_t* kpool;
  const half_t* vpool;
  const int* pos;
  const int* seq;
  const int* table_off;
  const int* tables;
  const int* tiles;  // (first token, rows) pairs
  int n_tiles, heads, kv_heads, block_size, bs_shift, xcd_heads;
  float scale_log2;
  half_t* out;
  int64_t out_stride;
};

__device__ __forceinline__ int kswz(int key) { return key & 7; }
__device__ __forceinline__ int vswz(int key) { return ((key >> 2) & 1) << 2; }

template <int D>
__global__ __launch_bounds__(kThreads, 2) void flash_prefill_kernel(const PrefillArgs a) {
  constexpr int CH = D / 8;                          // 16-byte chunks per row
  constexpr int MK = D / 16;                         // QK MFMAs per 32-key sub-tile
  constexpr int DT = D / 32;                         // 32-dim tiles of O^T
  constexpr int LOADS = kKeyTile * CH / kThreads;    // 16-byte chunks per thread per tile (each of K, V)

  __shared__ __attribute__((aligned(16))) half_t sK[kKeyTile * D];
  __shared__ __attribute__((aligned(16))) half_t sV[kKeyTile * D];

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = lane & 31, hh = lane >> 5;

  // Workgroup -> (tile, head): heaviest tiles first; per-XCD head ranges.
  const int b = blockIdx.x;
  int tile, head;
  if (a.xcd_heads > 0) {
    const int xcd = b & 7, s = b >> 3;
    tile = s / a.xcd_heads;
    head = xcd * a.xcd_heads + s % a.xcd_heads;
  } else {
    tile = b / a.heads;
    head = b % a.heads;
  }
  if (tile >= a.n_tiles) return;
  const int t0 = a.tiles[2 * tile], nrows = a.tiles[2 * tile + 1];
  const int kvh = head / (a.heads / a.kv_heads);
  const int p0 = a.pos[t0];
  const int* table = a.tables + a.table_off[a.seq[t0]];
  const int nkeys = p0 + nrows;
  const int bs = a.block_size, sh = a.bs_shift;

  // This wave's rows.
  const int row = w * 32 + c;
  const bool row_ok = row < nrows;
  const bool wave_on = w * 32 < nrows;
  const int qpos = p0 + row;
  const int wave_last = p0 + min(w * 32 + 31, nrows - 1);

  half8 qb[MK];
#pragma unroll
  for (int m = 0; m < MK; ++m) {
    if (row_ok) {
      qb[m] = load_half8(a.q + static_cast<int64_t>(t0 + row) * a.q_stride + static_cast<int64_t>(head) * D + 16 * m + 8 * hh);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) qb[m][e] = 0;
    }
  }

  float16v o[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[i][r] = 0.0f;
  float m_run = -INFINITY, l_part = 0.0f;
  const float cl = a.scale_log2;

  // Prefetch registers for one K/V tile.
  half8 kreg[LOADS], vreg[LOADS];
  auto load_tile = [&](int k0) {
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int ci = threadIdx.x + i * kThreads;
      const int kl = ci / CH, cc = ci % CH;
      const int key = k0 + kl;
      if (key < nkeys) {
        const int blk = table[sh >= 0 ? key >> sh : key / bs];
        const int slot = sh >= 0 ? key & (bs - 1) : key % bs;
        const int64_t off = kv_row_offset(blk, a.kv_heads, kvh, bs, slot, D) + 8 * cc;
        kreg[i] = load_half8(a.kpool + off);
        vreg[i] = load_half8(a.vpool + off);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          kreg[i][e] = 0;
          vreg[i][e] = 0;
        }
      }
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int ci = threadIdx.x + i * kThreads;
      const int kl = ci / CH, cc = ci % CH;
      *reinterpret_cast<half8*>(sK + kl * D + ((cc ^ kswz(kl)) << 3)) = kreg[i];
      *reinterpret_cast<half8*>(sV + kl * D + ((cc ^ vswz(kl)) << 3)) = vreg[i];
    }
  };

  load_tile(0);
  for (int k0 = 0; k0 < nkeys; k0 += kKeyTile) {
    __syncthreads();  // the previous tile's readers are done
    store_tile();
    __syncthreads();
    if (k0 + kKeyTile < nkeys) load_tile(k0 + kKeyTile);

#pragma unroll
    for (int sub = 0; sub < kKeyTile / 32; ++sub) {
      const int kb = k0 + 32 * sub;
      if (!wave_on || kb > wave_last) continue;  // uniform per wave
      float16v s;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = 0.0f;
#pragma unroll
      for (int m = 0; m < MK; ++m) {
        const int kl = 32 * sub + c;
        const half8 ka = *reinterpret_cast<const half8*>(sK + kl * D + (((2 * m + hh) ^ kswz(kl)) << 3));
        s = mfma32x32x16(ka, qb[m], s);
      }
      // Causal mask (and keys past the chunk, which are past every row).
      const bool need_mask = kb + 31 > p0 + w * 32;
      float mx = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kb + 8 * (r >> 2) + 4 * hh + (r & 3);
        if (need_mask && key > qpos) s[r] = -INFINITY;
        mx = fmaxf(mx, s[r]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_run, mx);
      const float base = m_new == -INFINITY ? 0.0f : m_new * cl;
      const float alpha = m_run == -INFINITY ? 0.0f : fast_exp2(m_run * cl - base);
      half8 pb[2];
      float psum = 0.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2(__builtin_fmaf(s[r], cl, -base));
        psum += p;
        pb[r >> 3][r & 7] = static_cast<half_t>(p);
      }
      l_part = l_part * alpha + psum;
      // Rescale O^T only if some row's running maximum changed.
      if (__ballot(m_new != m_run) != 0) {
#pragma unroll
        for (int i = 0; i < DT; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[i][r] *= alpha;
      }
      m_run = m_new;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int d = 32 * dt + c;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          half8 va;
#pragma unroll
          for (int sl = 0; sl < 8; ++sl) {
            const int kl = 32 * sub + 16 * u + 8 * (sl >> 2) + 4 * hh + (sl & 3);
            va[sl] = sV[kl * D + (((d >> 3) ^ vswz(kl)) << 3) + (d & 7)];
          }
          o[dt] = mfma32x32x16(va, pb[u], o[dt]);
        }
      }
    }
  }

  if (!row_ok) return;
  const float l_tot = l_part + __shfl_xor(l_part, 32);
  const float inv = 1.0f / l_tot;
  half_t* orow = a.out + static_cast<int64_t>(t0 + row) * a.out_stride + static_cast<int64_t>(head) * D;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      half4 v;
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = static_cast<half_t>(o[dt][4 * r4 + j] * inv);
      *reinterpret_cast<half4*>(orow + 32 * dt + 8 * r4 + 4 * hh) = v;
    }
}

}  // namespace
}  // namespace relay_hip

using namespace relay_hip;

extern "C" int rh_prefill_tile_rows(void) { return kRows; }

extern "C" int rh_flash_prefill(const void* q, int64_t q_row_stride, const void* kpool, const void* vpool,
                                const int* pos, const int* seq, const int* table_off, const int* tables,
                                const int* tiles, int n_tiles, int heads, int kv_heads, int head_dim, int block_size,
                                float scale, void* out, int64_t out_row_stride, void* stream) {
  if (n_tiles == 0) return 0;
  RH_REQUIRE(n_tiles > 0 && heads > 0 && kv_heads > 0 && heads % kv_heads == 0, "flash prefill: bad head counts");
  RH_REQUIRE(head_dim == 64 || head_dim == 128, "flash prefill: head_dim must be 64 or 128");
  RH_REQUIRE(block_size > 0, "flash prefill: bad block size");
  RH_REQUIRE(q_row_stride % 8 == 0 && out_row_stride % 4 == 0, "flash prefill: rows must be aligned");
  RH_REQUIRE((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(kpool) |
              reinterpret_cast<uintptr_t>(vpool)) % 16 == 0 &&
                 reinterpret_cast<uintptr_t>(out) % 8 == 0,
             "flash prefill: q, pools and out must be aligned");
  PrefillArgs a;
  a.q = static_cast<const half_t*>(q);
  a.q_stride = q_row_stride;
  a.kpool = static_cast<const half_t*>(kpool);
  a.vpool = static_cast<const half_t*>(vpool);
  a.pos = pos;
  a.seq = seq;
  a.table_off = table_off;
  a.tables = tables;
  a.tiles = tiles;
  a.n_tiles = n_tiles;
  a.heads = heads;
  a.kv_heads = kv_heads;
  a.block_size = block_size;
  a.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz(block_size) : -1;
  a.xcd_heads = heads % 8 == 0 ? heads / 8 : 0;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.out = static_cast<half_t*>(out);
  a.out_stride = out_row_stride;
  const int grid = n_tiles * heads;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (head_dim == 64) {
    RH_TRY_LAUNCH(hipLaunchKernelGGL(flash_prefill_kernel<64>, dim3(grid), dim3(kThreads), 0, s, a));
  } else {
    RH_TRY_LAUNCH(hipLaunchKernelGGL(flash_prefill_kernel<128>, dim3(grid), dim3(kThreads), 0, s, a));
  }
  return 0;
}
