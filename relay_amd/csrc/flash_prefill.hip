// Flash prefill attention over the paged KV cache for gfx950 (fp16 MFMA, fp32 softmax).
//
// The role of relay's flash_prefill_kernel<D> (cuda_kernels.cuh:28-178): causal attention of
// a chunk's query rows against keys 0 .. (row position), all read through the block table
// (a chunk at an offset sees the earlier chunks' keys). Re-cut for 64-wide waves and 32x32
// matrix cores:
//
// - Work unit: one workgroup of eight waves per (work item, query head). A work item is a
//   block of up to 128 consecutive rows of one chunk, or a pair of blocks (i, n-1-i) of
//   the same chunk processed one after the other, so that every workgroup does the same
//   causal work (rh_prefill_plan makes the items; it pairs when the grid is large).
// - Waves r and r+4 (the two waves of one SIMD) own the block's rows 32r .. 32r+31 and
//   split every key tile (128 keys at head_dim 64, 64 at 128): the first half goes to wave
//   r, the second to wave r+4. Each keeps its own running offset, sum and O^T; at the end of
//   the block wave r+4 hands them to wave r through LDS. So two waves stay busy on every SIMD
//   until the block's last tile (with one wave per 32-row strip, every SIMD drops to one wave
//   once the short blocks finish), and each SIMD holds one wave of each half (the second
//   halves carry more of the diagonal's work).
// - The workgroup walks the keys 0 .. (block's last position) a tile at a time: each tile
//   of K and V is gathered through the block table into registers one tile ahead (its block
//   ids another tile ahead) and written to one of two LDS buffers (one barrier per tile).
// - Per wave and half tile (one or two 32-key sub-steps, whose S^T chains interleave):
//     S^T[32 keys x 32 rows] = K[32 keys x D] * Q^T[D x 32 rows] - ref  (D/16 MFMA 32x32x16)
//   with q scaled into the exp2 domain (softmax scale * log2 e) and the accumulators
//   starting at minus the row's reference offset, so P = exp2(S^T) as it stands; a tile is
//   accepted while no lane's row sum passes 2^15 (no fp16 overflow) and otherwise redone
//   with the row maximum (new offset, O^T and sum rescaled) — a few tiles per row. Row sums
//   from the fp16 P values with packed dot products;
//     O^T[D x 32 rows] += V^T[D x 16 keys] * P^T[16 keys x 32 rows]     (D/32 MFMA 32x32x16)
//   The S^T accumulators are the P^T B operands as they stand. Lane (c, h) of S^T holds
//   keys {4h..4h+3, 8+4h..8+4h+3} of each 16-key group: two runs of 4 consecutive keys,
//   which is what one gfx950 transposing LDS read (ds_read_b64_tr_b16) returns from a
//   row-major V. So V is stored like K, and each V^T A operand is two such reads (the
//   earlier layout, V stored transposed with 4-byte writes of key pairs, spent more LDS
//   cycles on the writes than on all other LDS work together).
// - LDS rows (K and V) are XOR-swizzled in 16-byte chunks by key (kswz), so a read of 32
//   keys at one column spreads over the banks.
// - When the head count is a multiple of 8, each XCD (workgroup ids are dealt round-robin
//   over the 8 XCDs) gets a contiguous range of heads, i.e. few KV heads, so its L2 holds
//   the K/V its workgroups re-read.
#include <algorithm>
#include <cstring>
#include <type_traits>
#include <vector>

#include "../../include/relay_hip.h"
#include "common.h"

namespace relay_hip {
namespace {

constexpr int kRows = 128;    // query rows per block
constexpr int kWaves = 8;     // two per 32-row strip
constexpr int kThreads = kWaves * kWave;
// 32-key sub-steps per wave per tile: at D 64 two independent S^T chains per wave under
// one softmax (measured 45.0 -> 41.8 us at config 3); at D 128 the second chain's
// registers would spill.
template <int D>
constexpr int sub_steps() { return D == 128 ? 1 : 2; }

// One work item: block a (t0, rows, first position), block b likewise (rows 0: none), and
// the chunk's block-table offset. Layout of rh_prefill_plan's int32[8] records.
struct PrefillWork {
  int t0a, na, p0a, t0b, nb, p0b, table_off, pad;
};

struct PrefillArgs {
  const half_t* q;
  int64_t q_stride;
  const half_t* kpool;
  const half_t* vpool;
  const int* tables;
  const PrefillWork* work;
  int n_work, heads, kv_heads, block_size, bs_shift, xcd_heads;
  float scale_log2;
  half_t* out;
  int64_t out_stride;
};

// The value of lane l ^ 32 combined with lane l's, through one permlane32 swap (no LDS).
__device__ __forceinline__ float xlane_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __builtin_fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xlane_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]) - x;
}

// 16-byte chunk swizzle of K and V rows by key, chosen so that none of the kernel's LDS
// accesses has a bank conflict (64 banks of 4 bytes; a 16-byte access serves 16 lanes per
// cycle, an 8-byte one 32): the 16 lanes of a K operand read (keys c .. c+15 at one chunk)
// and the transposing V reads (4 consecutive keys x 4 chunks) each cover every bank once.
// Measured per instruction against key & 7 (key ^ key >> 3 at 128): K reads 8.2 -> 6.4
// clocks (16 -> 6.4 at head size 32), V reads at 128 8.0 -> 5.2; 2048-token prefill at
// head size 128 54.4 -> 52.6 us. Head size 64 keeps key & 7 (K reads 2-way conflicted):
// the conflict-free (key >> 1) & 7 measured 31.1 -> 31.8 us there.
template <int D>
__device__ __forceinline__ int kswz(int key) {
  return D == 128 ? ((key & 3) << 2) | ((key >> 2) & 3) : D == 64 ? key & 7 : (key >> 2) & 3;
}

// D is the compute width, DR the head size of the cache rows, q and out: equal, except head
// size 16, which runs at width 32 with dims 16..31 of K, V and q taken as zero.
template <int D, int DR, bool POW2>
__global__ __launch_bounds__(kThreads) void flash_prefill_kernel(const PrefillArgs a) {
  static_assert(DR == D || (DR == 16 && D == 32), "head size 16 runs at width 32");
  constexpr int kSub = sub_steps<D>();      // 32-key sub-steps per wave per tile
  constexpr int kKeyTile = 64 * kSub;       // keys per LDS tile
  constexpr int CH = D / 8;                                 // 16-byte chunks per row
  constexpr int MK = D / 16;                                // QK MFMAs per half tile
  constexpr int DT = D / 32;                                // 32-dim tiles of O^T
  constexpr int ITEMS = kKeyTile / 2 * CH;                  // (key pair, chunk) items per tile
  constexpr int PAIRS = (ITEMS + kThreads - 1) / kThreads;  // per thread
  constexpr int LOADS = 2 * PAIRS;                          // rows per thread per tile, each of K and V
  constexpr int KBUF = kKeyTile * D, VBUF = D * kKeyTile;   // halves per buffer
  constexpr int XSTRIP = DT * 16 * 64 + 2 * 64;             // floats per strip for the merge
  constexpr int SMEM = std::max(2 * KBUF + 2 * VBUF, 2 * 4 * XSTRIP);

  // Two K and two V buffers (row-major, 16-byte chunks XOR-swizzled by key); reused for the
  // merge of the half-tile partials.
  __shared__ __attribute__((aligned(16))) half_t smem[SMEM];
  half_t* const sK = smem;
  half_t* const sV = smem + 2 * KBUF;

  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 31, hh = lane >> 5;
  const int strip = w & 3, half = w >> 2;

  // Workgroup -> (work item, head).
  const int b = blockIdx.x;
  int wi, head;
  if (a.xcd_heads > 0) {
    const int xcd = b & 7, s = b >> 3;
    wi = s / a.xcd_heads;
    head = xcd * a.xcd_heads + s % a.xcd_heads;
  } else {
    wi = b / a.heads;
    head = b % a.heads;
  }
  if (wi >= a.n_work) return;
  const PrefillWork wk = a.work[wi];
  const int kvh = head / (a.heads / a.kv_heads);
  const int* table = a.tables + wk.table_off;
  const int bs = a.block_size, sh = a.bs_shift;
  const float cl = a.scale_log2;

  // Block-table lookups and K/V rows in flight for the tile after the one in LDS.
  int blk[LOADS];
  half8 kreg[LOADS], vreg[LOADS];
  // Row i of this thread: key p + (i & 1) * (tile / 2) of the tile, 16-byte chunk cc (valid
  // if < ITEMS); one load or LDS store instruction covers consecutive keys, i.e. both halves
  // of the LDS banks (a key row is 128 bytes at head size 64).
  auto item = [&](int i, int& kl, int& cc) {
    const int qi = threadIdx.x + (i >> 1) * kThreads;
    cc = qi % CH;
    kl = qi / CH + (i & 1) * (ITEMS / CH);
    return ITEMS % kThreads == 0 || qi < ITEMS;
  };

  for (int phase = 0; phase < 2; ++phase) {
    const int t0 = phase ? wk.t0b : wk.t0a, nrows = phase ? wk.nb : wk.na, p0 = phase ? wk.p0b : wk.p0a;
    if (nrows <= 0) break;
    const int nkeys = p0 + nrows;
    const int row = strip * 32 + c;
    const bool row_ok = row < nrows;
    const bool wave_on = strip * 32 < nrows;
    const int qpos = p0 + row;
    const int wave_last = p0 + min(strip * 32 + 31, nrows - 1);  // last key any row of the strip sees

    auto lookup = [&](int k0) {
#pragma unroll
      for (int i = 0; i < LOADS; ++i) {
        int kl, cc;
        if (item(i, kl, cc)) {
          // Keys past the block's last are masked for every row; read a valid row instead.
          const int key = min(k0 + kl, nkeys - 1);
          blk[i] = table[POW2 ? key >> sh : key / bs];
        }
      }
    };
    auto fetch = [&](int k0) {
#pragma unroll
      for (int i = 0; i < LOADS; ++i) {
        int kl, cc;
        if (item(i, kl, cc)) {
          const int key = min(k0 + kl, nkeys - 1);
          const int slot = POW2 ? key & (bs - 1) : key % bs;
          const int64_t off = kv_row_offset(blk[i], a.kv_heads, kvh, bs, slot, DR) + 8 * cc;
          if (DR == D || 8 * cc < DR) {
            kreg[i] = load_half8(a.kpool + off);
            vreg[i] = load_half8(a.vpool + off);
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) kreg[i][e] = vreg[i][e] = 0;
          }
        }
      }
    };
    auto store = [&](int buf) {
#pragma unroll
      for (int i = 0; i < LOADS; ++i) {
        int kl, cc;
        if (item(i, kl, cc)) {
          const int off = kl * D + ((cc ^ kswz<D>(kl)) << 3);
          *reinterpret_cast<half8*>(sK + buf * KBUF + off) = kreg[i];
          // V row-major like K (the PV operands come out of LDS through transposing reads).
          *reinterpret_cast<half8*>(sV + buf * VBUF + off) = vreg[i];
        }
      }
    };

    // q rows as MFMA B operands, scaled into the exp2 domain (scale * log2 e) on the way in:
    // exact when the caller already folded the scale into q (cl == 1), one more fp16
    // rounding of q otherwise.
    half8 qb[MK];
#pragma unroll
    for (int m = 0; m < MK; ++m) {
      if (row_ok && (DR == D || 16 * m + 8 * hh < DR)) {
        qb[m] = load_half8(a.q + static_cast<int64_t>(t0 + row) * a.q_stride + static_cast<int64_t>(head) * DR +
                           16 * m + 8 * hh);
#pragma unroll
        for (int e = 0; e < 8; ++e) qb[m][e] = static_cast<half_t>(static_cast<float>(qb[m][e]) * cl);
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
    // Row state (lane = row, shared by lanes c and c + 32): ref, the exp2-domain offset of
    // the row's O and sum (-inf until the row has seen a finite score); l_part, this lane's
    // share of the sum. The S^T accumulators start at -ref (negref; 0 while ref is -inf), so
    // the MFMAs deliver s - ref and P = exp2(S^T) needs no per-score arithmetic.
    float ref = -INFINITY, l_part = 0.0f;
    float16v negref;
#pragma unroll
    for (int r = 0; r < 16; ++r) negref[r] = 0.0f;
    bool have_ref = false;  // wave-uniform: every row of the wave has a finite ref

    // This wave's 32 kSub keys of the tile in LDS buffer `buf` starting at key k0.
    // MASK: the keys cross a row of this strip (only the diagonal tiles); a separate
    // instantiation, because a uniform branch around the selects is if-converted into
    // per-element work on every tile.
    auto compute = [&](auto mask_tag, int buf, int kb) {
      constexpr bool MASK = decltype(mask_tag)::value;
      float16v s[kSub];
#pragma unroll
      for (int m = 0; m < MK; ++m)
#pragma unroll
        for (int j = 0; j < kSub; ++j) {
          const half_t* kt = sK + buf * KBUF + (32 * kSub * half + 32 * j + c) * D;
          const half8 ka = *reinterpret_cast<const half8*>(kt + (((2 * m + hh) ^ kswz<D>(c)) << 3));
          s[j] = mfma32x32x16(ka, qb[m], m == 0 ? negref : s[j]);
        }
      if (MASK) {
        const int lim = qpos - kb - 4 * hh;  // key offsets above this are masked
#pragma unroll
        for (int j = 0; j < kSub; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (32 * j + 8 * (r >> 2) + (r & 3) > lim) s[j][r] = -INFINITY;
      }
      half8 pb[2 * kSub];
      float psum = 0.0f;
      // Row sum of the fp16 P values (the ones the PV product uses), fp32 accumulation.
      auto exp_and_sum = [&](float shift) {
        psum = 0.0f;
#pragma unroll
        for (int j = 0; j < kSub; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            pb[2 * j + (r >> 3)][r & 7] = static_cast<half_t>(fast_exp2(s[j][r] - shift));
#pragma unroll
        for (int u = 0; u < 2 * kSub; ++u)
#pragma unroll
          for (int e = 0; e < 8; e += 2) {
            const half2_t p2 = {pb[u][e], pb[u][e + 1]};
            psum = __builtin_amdgcn_fdot2(p2, half2_t{1.0f16, 1.0f16}, psum, false);
          }
      };
      // Fast path: P = exp2(s - ref) as it stands, accepted while every lane's sum is at
      // most 2^15 (so no P overflows fp16; NaN and inf fail the test). The reference offset
      // only moves when a row's scores rise well above it, on a few tiles per row.
      bool slow = !have_ref;
      if (!slow) {
        exp_and_sum(0.0f);
        slow = __ballot(!(psum <= 32768.0f)) != 0;
      }
      if (slow) {
        // The row maximum (both lanes of the row), a new offset where it exceeds the old one
        // by more than 2^8, or where the row had none.
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < kSub; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = __builtin_fmaxf(mx, s[j][r]);
        mx = xlane_max(mx);
        float shift = 0.0f, alpha = 1.0f;
        if (ref == -INFINITY) {
          if (mx != -INFINITY) {
            shift = mx;
            ref = mx;
            alpha = 0.0f;
          }
        } else if (mx > 8.0f) {
          shift = mx;
          ref += mx;
          alpha = fast_exp2(-mx);
        }
        exp_and_sum(shift);
        l_part *= alpha;
        if (__ballot(alpha != 1.0f) != 0) {
#pragma unroll
          for (int i = 0; i < DT; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[i][r] *= alpha;
        }
        const float nr = ref == -INFINITY ? 0.0f : -ref;
#pragma unroll
        for (int r = 0; r < 16; ++r) negref[r] = nr;
        have_ref = __ballot(ref == -INFINITY) == 0;
      }
      l_part += psum;
      // V^T operand of lane (d, hh) for pb[u]: slots e < 4 hold keys kr .. kr + 3 and slots
      // e >= 4 keys kr + 8 .. kr + 11 (the S^T accumulator order), kr = 32 (u / 2) + 16 (u % 2)
      // + 4 hh; each run of 4 keys is one transposing read in which lane i16 of the 16-lane
      // group reads row kr + i16 / 4, columns d0 + 4 (i16 % 4) .. +3.
      const int i16 = lane & 15;
#pragma unroll
      for (int u = 0; u < 2 * kSub; ++u)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const int col = 32 * dt + 16 * ((lane >> 4) & 1) + 4 * (i16 & 3);
          const int kr = 32 * kSub * half + 32 * (u >> 1) + 16 * (u & 1) + 4 * hh + (i16 >> 2);
          const half_t* vb = sV + buf * VBUF + (col & 7);
          const half4 lo = tr_read_b64(vb + kr * D + (((col >> 3) ^ kswz<D>(kr)) << 3));
          const half4 hi = tr_read_b64(vb + (kr + 8) * D + (((col >> 3) ^ kswz<D>(kr + 8)) << 3));
          const half8 va = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          o[dt] = mfma32x32x16(va, pb[u], o[dt]);
        }
    };

    // Tile j lives in LDS buffer j & 1. Step j: store tile j+1 (rows fetched a step ago)
    // into the other buffer, issue tile j+2's loads and tile j+3's block ids, compute
    // tile j, barrier; the loads are in flight under the compute.
    const int ntiles = (nkeys + kKeyTile - 1) / kKeyTile;
    __syncthreads();  // the previous phase's merge is done with the LDS
    lookup(0);
    fetch(0);
    if (ntiles > 1) lookup(kKeyTile);
    store(0);
    if (ntiles > 1) fetch(kKeyTile);
    if (ntiles > 2) lookup(2 * kKeyTile);
    __syncthreads();
    const int first_masked = p0 + strip * 32 - 32 * kSub * (half + 1) + 1;  // unmasked: j * kKeyTile <= this
    const int j_mask = min(ntiles, first_masked >= 0 ? first_masked / kKeyTile + 1 : 0);
    auto prepare = [&](int j) {
      if (j + 1 < ntiles) store((j + 1) & 1);
      if (j + 2 < ntiles) fetch((j + 2) * kKeyTile);
      if (j + 3 < ntiles) lookup((j + 3) * kKeyTile);
    };
    int j = 0;
    for (; j < j_mask; ++j) {
      prepare(j);
      if (wave_on) compute(std::false_type{}, j & 1, j * kKeyTile + 32 * kSub * half);
      __syncthreads();
    }
    for (; j < ntiles; ++j) {
      prepare(j);
      const int kb = j * kKeyTile + 32 * kSub * half;
      if (wave_on && kb <= wave_last) compute(std::true_type{}, j & 1, kb);  // uniform per wave
      __syncthreads();
    }

    // Merge the strip's two halves: the odd wave's (max, sum, O^T) through LDS (the tile
    // buffers are free after the loop's last barrier).
    float* const xo = reinterpret_cast<float*>(smem) + strip * XSTRIP;
    float* const xml = xo + DT * 16 * 64;
    if (half) {
#pragma unroll
      for (int i = 0; i < DT; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) xo[(i * 16 + r) * 64 + lane] = o[i][r];
      xml[lane] = ref;
      xml[64 + lane] = l_part;
    }
    __syncthreads();
    if (!half && row_ok) {
      // The even wave saw key 0, so its offset is finite; the odd one's may not be.
      const float m_b = xml[lane], l_b = xml[64 + lane];
      const float m = fmaxf(ref, m_b);
      const float fa = fast_exp2(ref - m);
      const float fb = m_b == -INFINITY ? 0.0f : fast_exp2(m_b - m);
      const float l = l_part * fa + l_b * fb;
      const float inv = 1.0f / (l + xlane_sum(l));
      half_t* orow = a.out + static_cast<int64_t>(t0 + row) * a.out_stride + static_cast<int64_t>(head) * DR;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          half4 v;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int r = 4 * r4 + j;
            v[j] = static_cast<half_t>((o[dt][r] * fa + xo[(dt * 16 + r) * 64 + lane] * fb) * inv);
          }
          if (DR == D || 32 * dt + 8 * r4 + 4 * hh < DR) *reinterpret_cast<half4*>(orow + 32 * dt + 8 * r4 + 4 * hh) = v;
        }
    }
  }
}

template <int D, int DR>
int launch(const PrefillArgs& a, hipStream_t s) {
  const int grid = a.n_work * a.heads;
  if (a.bs_shift >= 0) {
    RH_TRY_LAUNCH(hipLaunchKernelGGL((flash_prefill_kernel<D, DR, true>), dim3(grid), dim3(kThreads), 0, s, a));
  } else {
    RH_TRY_LAUNCH(hipLaunchKernelGGL((flash_prefill_kernel<D, DR, false>), dim3(grid), dim3(kThreads), 0, s, a));
  }
  return 0;
}

}  // namespace
}  // namespace relay_hip

using namespace relay_hip;

extern "C" int rh_prefill_tile_rows(void) { return kRows; }

extern "C" int rh_prefill_plan(const int* chunk_t0, const int* chunk_rows, const int* chunk_pos0,
                               const int* chunk_table_off, int n_chunks, int heads, int* work, int capacity) {
  RH_REQUIRE(n_chunks >= 0 && heads > 0 && capacity >= 0, "prefill plan: bad arguments");
  long blocks = 0;
  for (int s = 0; s < n_chunks; ++s) {
    RH_REQUIRE(chunk_rows[s] >= 0 && chunk_pos0[s] >= 0, "prefill plan: negative rows or position");
    blocks += (chunk_rows[s] + kRows - 1) / kRows;
  }
  // Pair blocks only when the unpaired grid fills the GPU (256 CUs) twice over; otherwise
  // the halved grid would leave CUs idle.
  const bool pair = blocks * heads >= 512;
  std::vector<std::pair<long, PrefillWork>> items;
  auto cost = [](int rows, int p0) { return static_cast<long>(rows) * (p0 + rows); };
  for (int s = 0; s < n_chunks; ++s) {
    const int n = chunk_rows[s], nb = (n + kRows - 1) / kRows;
    auto blk = [&](int i, int& t0, int& rows, int& p0) {
      t0 = chunk_t0[s] + i * kRows;
      rows = std::min(kRows, n - i * kRows);
      p0 = chunk_pos0[s] + i * kRows;
    };
    for (int i = 0, j = nb - 1; i <= j; ++i, --j) {
      PrefillWork wk{};
      wk.table_off = chunk_table_off[s];
      blk(j, wk.t0a, wk.na, wk.p0a);  // the heavier block first
      long c = cost(wk.na, wk.p0a);
      if (i < j) {
        PrefillWork light = wk;
        blk(i, light.t0a, light.na, light.p0a);
        if (pair) {
          wk.t0b = light.t0a;
          wk.nb = light.na;
          wk.p0b = light.p0a;
          c += cost(wk.nb, wk.p0b);
        } else {
          items.push_back({cost(light.na, light.p0a), light});
        }
      }
      items.push_back({c, wk});
    }
  }
  RH_REQUIRE(static_cast<long>(items.size()) <= capacity, "prefill plan: work capacity too small");
  // Heaviest first: the dispatcher starts them first and the light ones fill in behind.
  std::stable_sort(items.begin(), items.end(), [](const auto& x, const auto& y) { return x.first > y.first; });
  for (std::size_t i = 0; i < items.size(); ++i) std::memcpy(work + 8 * i, &items[i].second, sizeof(PrefillWork));
  return static_cast<int>(items.size());
}

extern "C" int rh_flash_prefill(const void* q, int64_t q_row_stride, const void* kpool, const void* vpool,
                                const int* tables, const int* work, int n_work, int heads, int kv_heads, int head_dim,
                                int block_size, float scale, void* out, int64_t out_row_stride, void* stream) {
  if (n_work == 0) return 0;
  RH_REQUIRE(n_work > 0 && heads > 0 && kv_heads > 0 && heads % kv_heads == 0, "flash prefill: bad head counts");
  RH_REQUIRE(head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128,
             "flash prefill: head_dim must be 16, 32, 64 or 128");
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
  a.tables = tables;
  a.work = reinterpret_cast<const PrefillWork*>(work);
  a.n_work = n_work;
  a.heads = heads;
  a.kv_heads = kv_heads;
  a.block_size = block_size;
  a.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz(block_size) : -1;
  a.xcd_heads = heads % 8 == 0 ? heads / 8 : 0;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.out = static_cast<half_t*>(out);
  a.out_stride = out_row_stride;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (head_dim) {
    case 16: return launch<32, 16>(a, s);
    case 32: return launch<32, 32>(a, s);
    case 64: return launch<64, 64>(a, s);
    default: return launch<128, 128>(a, s);
  }
}
