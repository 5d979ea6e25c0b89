// Split-context paged decode attention for gfx950, with the log-sum-exp merge fused in.
//
// Work unit: one workgroup per (decode token, kv head, 16-head chunk of its query group,
// slice of `slice_keys` context keys) -- the split of relay's decode_attention_kernel
// (cuda_kernels.cuh:180-339). The slice is cut into chunks of 16 KB of K+V (64 keys at
// head_dim 64, 32 at 128) dealt round-robin to the workgroup's 4 or 8 waves. Per chunk a
// wave issues every K and V load first (16 KB in flight per wave, 128 KB per 8-wave
// workgroup), then walks the chunk in steps of 32 keys (measured: 16 KB chunks stream
// faster than 32 KB ones, whose registers also cap a CU at 8 waves):
//
//   S^T[16 keys x 16 heads] = K[16 keys x D] * Q^T[D x 16 heads]     (MFMA 16x16x32, D/32 per tile)
//   online softmax per head in the log2 domain, per lane (lane = head column)
//   O^T[D x 16 heads] += V^T[D x 32 keys] * P^T[32 keys x 16 heads]   (MFMA 16x16x32, D/16 tiles)
//
// All query heads of the group share one read of each K and V row (relay's kernel does
// this with a G-head loop per thread; here the heads are MFMA columns, so the score
// arithmetic costs no vector-ALU time and the kernel stays bound by HBM).
// K rows go straight from global memory into MFMA A operands: lane (c, g) loads key c of
// the tile, dims [8g, 8g+8) of each 32-wide group -- one 16-byte load. P^T comes out of
// the S^T accumulators already in B-operand order (the k slots of the PV product are a
// permutation of the 32 keys, the same for A and B). V needs the transpose V^T, which goes
// through LDS: each lane writes 16-byte row chunks, then reads single halves in column
// order; chunks are XOR-swizzled by key so the 4 key groups of a read hit disjoint banks.
//
// Metadata: the host packs, per decode token, (token row, context length, offset of its
// block table) -- the facts relay's kernel reaches through pos/seq/table_off
// (cuda_kernels.cuh:16-26, 236-250) -- so a workgroup needs one scalar load before it can
// read the block table. With a power-of-two block size >= 16 every 16-key tile lies in
// one block, so its table entry is wave-uniform and read by the scalar unit; other block
// sizes look entries up per lane. Keys past the context are masked (scores -inf, V rows
// zeroed).
//
// Merging: the waves of a workgroup merge in LDS. When a sequence has several slices, the
// last of its workgroups to finish merges them (an atomic counter per group; the partials
// travel through agent-coherent sc1 stores and loads, so no cache-wide fence is needed):
// no second kernel launch. Slice partials are (M, L) in the log2 domain plus the
// unnormalized O. Workgroup ids are mapped so the slices of one group land on one XCD
// (ids are dealt round-robin over the 8 XCDs).
#include <algorithm>
#include <mutex>
#include <string>

#include "../../include/relay_hip.h"
#include "common.h"

namespace relay_hip {
namespace {

constexpr int kStepKeys = 32;

struct DecodeArgs {
  const half_t* q;
  int64_t q_stride;
  const half_t* kpool;
  const half_t* vpool;
  const int4* dec_meta;  // per decode token: (token row, context, table offset, unused)
  const int* tables;
  int heads, kv_heads, group, hchunks, block_size, bs_shift, slice, max_parts, groups_total;
  float scale_log2;
  float* part_o;
  float* part_ml;
  int* counters;
  half_t* out;
  int64_t out_stride;
};

// Slices merged with all their loads issued together (more take a plain loop).
constexpr int kMergeBatch = 8;

// Swizzle of a key's 16-byte chunks in the V staging rows (within the row's D / 8 chunks).
template <int D>
__device__ __forceinline__ int vswz(int key) {
  return D >= 64 ? ((key >> 2) & 3) << 1 : ((key >> 2) & 1) << 1;
}

// Keys per streaming stage of a wave: 16 KB of K+V at head sizes 64 and 128, 8 KB at 32
// (also the compute width of head size 16).
template <int D>
constexpr int stage_keys() {
  return D == 64 ? 64 : D == 128 ? 32 : 128;
}

// One chunk of a wave's K and V in registers.
template <int D>
struct Stage {
  static constexpr int STEPS = stage_keys<D>() / kStepKeys;
  static constexpr int KH = D / 32;
  static constexpr int VL = kStepKeys * (D / 8) / kWave;
  half8 k[STEPS][2][KH];
  half8 v[STEPS][VL];
};

// SCALAR: block_size is a power of two >= 16 (table entries are wave-uniform per tile).
// D is the compute width, DR the head size of the cache rows, q and out: equal, except head
// size 16, which runs at width 32 with dims 16..31 of K, V and q taken as zero.
// Occupancy: up to D = 64 the kernel fits 128 VGPRs, so a CU holds two 8-wave workgroups
// (4 waves per SIMD); at D = 128 it needs more and holds one.
template <int D, int DR, int WAVES, bool SCALAR>
__global__ __launch_bounds__(WAVES * kWave) __attribute__((amdgpu_waves_per_eu(D <= 64 ? 4 : 2, D <= 64 ? 4 : 2))) void paged_decode_kernel(
    const DecodeArgs a) {
  constexpr int SK = stage_keys<D>();
  constexpr int STEPS = SK / kStepKeys;
  constexpr int CH = D / 8;                         // 16-byte chunks per row
  constexpr int KH = D / 32;                        // 32-wide dim groups (QK MFMAs per tile)
  constexpr int DT = D / 16;                        // 16-dim tiles of O^T
  constexpr int VL = kStepKeys * CH / kWave;        // V loads per lane per step
  constexpr int VKEYS = kWave / CH;                 // keys covered by one V load
  constexpr int NT = WAVES * kWave;
  static_assert(kStepKeys * D * 2 == 16 * D * 4, "the merge area reuses the V staging");
  static_assert(DR == D || (DR == 16 && D == 32), "head size 16 runs at width 32");

  __shared__ __attribute__((aligned(16))) half_t s_v[WAVES][kStepKeys * D];
  __shared__ float s_m[WAVES][16], s_l[WAVES][16];
  __shared__ int s_last;

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, g = lane >> 4;

  // Workgroup -> (group, part), the slices of one group on one XCD.
  const int b = blockIdx.x;
  const int sl = b >> 3;
  const int part = sl % a.max_parts;
  const int grp = (sl / a.max_parts) * 8 + (b & 7);
  if (grp >= a.groups_total) return;
  const int per_tok = a.kv_heads * a.hchunks;
  const int di = grp / per_tok;
  const int kvh = (grp % per_tok) / a.hchunks, hc = grp % a.hchunks;
  const int4 meta = a.dec_meta[di];
  const int t = meta.x, ctx = meta.y;
  const int* table = a.tables + meta.z;
  const int nparts = (ctx + a.slice - 1) / a.slice;
  if (part >= nparts) return;
  const int begin = part * a.slice, end = min(ctx, begin + a.slice);
  const int h0 = kvh * a.group + hc * 16;
  const int nh = min(16, a.group - hc * 16);
  const int bs = a.block_size, sh = a.bs_shift, kvn = a.kv_heads;

  // End of the chunk being computed (keys at or past it are masked).
  int we_cur = begin;

  // Cache row (D elements) of the first slot of a block, for this kv head.
  auto block_row = [&](int blk) -> unsigned { return static_cast<unsigned>((blk * kvn + kvh) * bs); };
  // Row of position j (clamped into the context).
  auto row_any = [&](int j) -> unsigned {
    j = min(j, end - 1);
    return block_row(table[j / bs]) + static_cast<unsigned>(j % bs);
  };
  // Row of key (tile + off): tile is a 16-aligned wave-uniform position, off < 16 per lane;
  // the tile's block comes from one scalar table read.
  auto row_tile = [&](int tile, int off) -> unsigned {
    const int ts = min(tile, end - 1);
    const int slot = ts & (bs - 1);
    return block_row(table[ts >> sh]) + static_cast<unsigned>(min(slot + off, bs - 1));
  };
  // Issue every load of the chunk that starts at key k0 (rows first, then the loads).
  auto issue = [&](Stage<D>& st, int k0) {
    unsigned krow[STEPS][2], vrow[STEPS][VL];
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int ks = k0 + s * kStepKeys;
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) krow[s][tt] = SCALAR ? row_tile(ks + 16 * tt, c) : row_any(ks + 16 * tt + c);
#pragma unroll
      for (int i = 0; i < VL; ++i) {
        const int kk = VKEYS * i;  // first key of the load, relative to the step
        vrow[s][i] = SCALAR ? row_tile(ks + (kk & ~15), (kk & 15) + lane / CH) : row_any(ks + kk + lane / CH);
      }
    }
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int h = 0; h < KH; ++h)
          if (DR == D || 32 * h + 8 * g < DR) {
            st.k[s][tt][h] = load_half8(a.kpool + static_cast<int64_t>(krow[s][tt]) * DR + 32 * h + 8 * g);
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) st.k[s][tt][h][e] = 0;
          }
      // V rows as non-temporal loads (the nt policy; K keeps the default one). Measured: 32 x
      // 2048 at D64 18.2 -> 16.3 us (512-key slices), 17.7 -> 15.9 (1024); 48 x 8192 at D128
      // 280 -> 255 us. Both K and V non-temporal: 17.1, 17.9, 265; K alone 16.4, 16.9, 277.
#pragma unroll
      for (int i = 0; i < VL; ++i)
        if (DR == D || 8 * (lane % CH) < DR) {
          st.v[s][i] = __builtin_bit_cast(half8, __builtin_nontemporal_load(reinterpret_cast<const uint4v*>(
                                                     a.vpool + static_cast<int64_t>(vrow[s][i]) * DR + 8 * (lane % CH))));
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) st.v[s][i][e] = 0;
        }
    }
  };

  half_t* sv = s_v[w];
  float m_run = -INFINITY, l_part = 0.0f;
  float4v o[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) o[i] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
  half8 qb[KH];

  // Online softmax and PV for the chunk at k0 (keys at or past we_cur are masked).
  auto compute = [&](const Stage<D>& st, int k0) {
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int ks = k0 + s * kStepKeys;
      if (ks >= we_cur) break;
      // This step's V rows into the wave's staging area (swizzled 16-byte chunks); rows
      // past the range are zeroed (their weights are 0, their bytes may be anything).
#pragma unroll
      for (int i = 0; i < VL; ++i) {
        const int kl = VKEYS * i + lane / CH, cc = lane % CH;
        half8 v = st.v[s][i];
        if (ks + kl >= we_cur) {
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = 0;
        }
        *reinterpret_cast<half8*>(sv + kl * D + ((cc ^ vswz<D>(kl)) << 3)) = v;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

      float4v sc4[2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        sc4[tt] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int h = 0; h < KH; ++h) sc4[tt] = mfma16x16x32(st.k[s][tt][h], qb[h], sc4[tt]);
      }
      float sc[8];
      float mx = -INFINITY;
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = ks + 16 * tt + 4 * g + r;
          const float v = key < we_cur ? sc4[tt][r] * a.scale_log2 : -INFINITY;
          sc[tt * 4 + r] = v;
          mx = fmaxf(mx, v);
        }
      mx = group4_max(mx);
      const float m_new = fmaxf(m_run, mx);
      const float m_use = m_new == -INFINITY ? 0.0f : m_new;
      const float alpha = fast_exp2(m_run - m_use);
      half8 pt;
      float psum = 0.0f;
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const float p = fast_exp2(sc[r] - m_use);
        psum += p;
        pt[r] = static_cast<half_t>(p);
      }
      l_part = l_part * alpha + psum;
      m_run = m_new;

      // O^T += V^T P^T, V^T read column-wise from the staging rows.
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        // Transposing LDS reads: lane c of group g reads 8 bytes of V row (kb + c / 4),
        // columns 16 dt + 4 (c % 4) .. +3, and receives V[kb .. kb + 3][16 dt + c]; kb = 4g
        // and 16 + 4g give the operand's two runs of 4 keys.
        const int col = 16 * dt + 4 * (c & 3);
        const int k0r = 4 * g + (c >> 2), k1r = 16 + 4 * g + (c >> 2);
        const half4 lo = tr_read_b64(sv + k0r * D + (((col >> 3) ^ vswz<D>(k0r)) << 3) + (col & 7));
        const half4 hi = tr_read_b64(sv + k1r * D + (((col >> 3) ^ vswz<D>(k1r)) << 3) + (col & 7));
        const half8 vt = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        float4v acc = o[dt];
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] *= alpha;
        o[dt] = mfma16x16x32(vt, pt, acc);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  };

  // Q once; the first chunk's loads go out before it (Q is needed only at the first MFMA).
  bool have_q = false;
  for (int k0 = begin + w * SK; k0 < end; k0 += WAVES * SK) {
    Stage<D> st;
    issue(st, k0);
    if (!have_q) {
#pragma unroll
      for (int h = 0; h < KH; ++h) {
        if (c < nh && (DR == D || 32 * h + 8 * g < DR)) {
          qb[h] = load_half8(a.q + static_cast<int64_t>(t) * a.q_stride + static_cast<int64_t>(h0 + c) * DR + 32 * h +
                             8 * g);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) qb[h][e] = 0;
        }
      }
      have_q = true;
    }
    // All of the chunk's loads are in flight before any of its arithmetic.
    __builtin_amdgcn_sched_barrier(0);
    we_cur = min(end, k0 + SK);
    compute(st, k0);
  }
  const float l_tot = group4_sum(l_part);

  // Merge the waves' partials in LDS (the V staging area, now free).
  __syncthreads();
  // [wave][head][D], head hh's row rotated by 4 * hh floats: the 16 heads of one write
  // instruction would otherwise all hit the same LDS banks (a 16-way conflict that
  // serialised this store for ~1.7 us per workgroup).
  float* so = reinterpret_cast<float*>(&s_v[0][0]);
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r = 0; r < 4; ++r) so[(w * 16 + c) * D + ((16 * dt + 4 * g + 4 * c) & (D - 1)) + r] = o[dt][r];
  if (g == 0) {
    s_m[w][c] = m_run;
    s_l[w][c] = l_tot;
  }
  __syncthreads();

  const bool single = nparts == 1;
  for (int idx = threadIdx.x; idx < nh * DR; idx += NT) {
    const int hh = idx / DR, d = idx % DR;
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < WAVES; ++ww) M = fmaxf(M, s_m[ww][hh]);
    float L = 0.0f, O = 0.0f;
#pragma unroll
    for (int ww = 0; ww < WAVES; ++ww) {
      const float mw = s_m[ww][hh];
      if (mw != -INFINITY) {
        const float f = fast_exp2(mw - M);
        L += f * s_l[ww][hh];
        O += f * so[(ww * 16 + hh) * D + ((d + 4 * hh) & (D - 1))];
      }
    }
    if (single) {
      a.out[static_cast<int64_t>(t) * a.out_stride + static_cast<int64_t>(h0 + hh) * DR + d] = static_cast<half_t>(O / L);
    } else {
      const int64_t pb = (static_cast<int64_t>(di) * a.heads + h0 + hh) * a.max_parts + part;
      coherent_store(&a.part_o[pb * DR + d], O);
      if (d == 0) {
        coherent_store(&a.part_ml[pb * 2], M);
        coherent_store(&a.part_ml[pb * 2 + 1], L);
      }
    }
  }
  if (single) return;

  // The last workgroup of this group merges every slice. Waiting for this workgroup's
  // coherent stores to complete before the barrier orders them before the counter
  // increment; the merging workgroup reads the partials with coherent loads.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(&a.counters[grp], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = prev == nparts - 1;
    if (last) __hip_atomic_store(&a.counters[grp], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last;
  }
  __syncthreads();
  if (!s_last) return;
  for (int idx = threadIdx.x; idx < nh * DR; idx += NT) {
    const int hh = idx / DR, d = idx % DR;
    const int64_t base = (static_cast<int64_t>(di) * a.heads + h0 + hh) * a.max_parts;
    float M = -INFINITY, L = 0.0f, O = 0.0f;
    if (nparts <= kMergeBatch) {
      // Every partial's loads in flight at once (a loop of dependent loads costs one L2
      // round trip per load); same arithmetic, in the same order, as the general loop.
      float mv[kMergeBatch], lv[kMergeBatch], ov[kMergeBatch];
#pragma unroll
      for (int p = 0; p < kMergeBatch; ++p) {
        if (p < nparts) {
          mv[p] = coherent_load(&a.part_ml[(base + p) * 2]);
          lv[p] = coherent_load(&a.part_ml[(base + p) * 2 + 1]);
          ov[p] = coherent_load(&a.part_o[(base + p) * DR + d]);
        }
      }
#pragma unroll
      for (int p = 0; p < kMergeBatch; ++p)
        if (p < nparts) M = fmaxf(M, mv[p]);
#pragma unroll
      for (int p = 0; p < kMergeBatch; ++p) {
        if (p < nparts) {
          const float f = fast_exp2(mv[p] - M);
          L += f * lv[p];
          O += f * ov[p];
        }
      }
    } else {
      // The same arithmetic in the same order, with the loads of kMergeBatch slices issued
      // together in each round.
      for (int p0 = 0; p0 < nparts; p0 += kMergeBatch) {
        float mv[kMergeBatch];
#pragma unroll
        for (int q = 0; q < kMergeBatch; ++q)
          if (p0 + q < nparts) mv[q] = coherent_load(&a.part_ml[(base + p0 + q) * 2]);
#pragma unroll
        for (int q = 0; q < kMergeBatch; ++q)
          if (p0 + q < nparts) M = fmaxf(M, mv[q]);
      }
      for (int p0 = 0; p0 < nparts; p0 += kMergeBatch) {
        float mv[kMergeBatch], lv[kMergeBatch], ov[kMergeBatch];
#pragma unroll
        for (int q = 0; q < kMergeBatch; ++q) {
          if (p0 + q < nparts) {
            mv[q] = coherent_load(&a.part_ml[(base + p0 + q) * 2]);
            lv[q] = coherent_load(&a.part_ml[(base + p0 + q) * 2 + 1]);
            ov[q] = coherent_load(&a.part_o[(base + p0 + q) * DR + d]);
          }
        }
#pragma unroll
        for (int q = 0; q < kMergeBatch; ++q) {
          if (p0 + q < nparts) {
            const float f = fast_exp2(mv[q] - M);
            L += f * lv[q];
            O += f * ov[q];
          }
        }
      }
    }
    a.out[static_cast<int64_t>(t) * a.out_stride + static_cast<int64_t>(h0 + hh) * DR + d] = static_cast<half_t>(O / L);
  }
}

template <int D, int DR, int WAVES>
int launch(const DecodeArgs& a, int grid, hipStream_t s) {
  if (a.bs_shift >= 4) {
    RH_TRY_LAUNCH(
        hipLaunchKernelGGL((paged_decode_kernel<D, DR, WAVES, true>), dim3(grid), dim3(WAVES * kWave), 0, s, a));
  } else {
    RH_TRY_LAUNCH(
        hipLaunchKernelGGL((paged_decode_kernel<D, DR, WAVES, false>), dim3(grid), dim3(WAVES * kWave), 0, s, a));
  }
  return 0;
}

template <int D, int DR>
int launch_waves(const DecodeArgs& a, int grid, bool eight, hipStream_t s) {
  return eight ? launch<D, DR, 8>(a, grid, s) : launch<D, DR, 4>(a, grid, s);
}

}  // namespace
}  // namespace relay_hip

using namespace relay_hip;

extern "C" int rh_decode_chunk_keys(int head_dim) {
  switch (head_dim) {
    case 16:
    case 32: return stage_keys<32>();
    case 64: return stage_keys<64>();
    case 128: return stage_keys<128>();
    default: return -1;
  }
}

extern "C" int rh_decode_slice_keys(int n_dec, int kv_heads, int group, int head_dim, int max_ctx) {
  const int chunk = rh_decode_chunk_keys(head_dim);
  if (chunk <= 0 || n_dec <= 0 || max_ctx <= 0) return chunk;
  // Measured on MI355X (1 x 640 / D64 up to 48 x 8192 / D128), otherwise: one slice for at most 16
  // (context, kv head) groups of at most 16 chunks; otherwise at least two slices per
  // context (enough workgroups to spread over the 256 CUs), more while there are fewer
  // than 256 groups, but never below 8 chunks (one per wave of an 8-wave workgroup).
  const long groups = static_cast<long>(n_dec) * kv_heads * ((group + 15) / 16);
  // Head size 64 or 128 with few groups: the step is latency-bound, so kMergeBatch slices
  // per context (the merge then takes one round of loads), of 2 to 8 chunks, as long as that
  // makes at most 256 workgroups (longer contexts take the rule below: enough workgroups
  // to stream from HBM); the launcher gives them 8 waves from 4 chunks on.
  // Measured (us, against the earlier 4-chunk minimum on 4 waves): 1 x 640 keys, 9/3 heads
  // (config 1) 6.87 -> 6.16; 1 x 2048, 32/4 8.57 -> 8.12; 8 x 2048, 32/4 10.78 -> 10.19;
  // 1 x 2048, 32/8, D128 11.65 -> 10.41.
  if (head_dim == 64 || head_dim == 128) {
    const long small = std::max(2L * chunk, static_cast<long>((max_ctx + kMergeBatch * chunk - 1) / (kMergeBatch * chunk) * chunk));
    if (small <= 8L * chunk && groups * ((max_ctx + small - 1) / small) <= 256) return static_cast<int>(small);
  }
  // A handful of short contexts: one slice (no merge); the launch is latency-bound anyway.
  if (groups <= 16 && max_ctx <= 16 * chunk) return (max_ctx + chunk - 1) / chunk * chunk;
  const long parts = std::max(2L, 256 / groups);
  const long per_part = (max_ctx + parts - 1) / parts;
  const long keys = std::max(8L * chunk, (per_part + chunk - 1) / chunk * chunk);
  return static_cast<int>(keys);
}

extern "C" int rh_paged_decode_attention(const void* q, int64_t q_row_stride, const void* kpool, const void* vpool,
                                         const int* dec_meta, const int* tables, int n_dec, int heads, int kv_heads,
                                         int head_dim, int block_size, int slice_keys, int max_parts, float scale,
                                         float* part_o, float* part_ml, int* counters, void* out,
                                         int64_t out_row_stride, void* stream) {
  if (n_dec == 0) return 0;
  RH_REQUIRE(n_dec > 0 && heads > 0 && kv_heads > 0 && heads % kv_heads == 0, "decode attention: bad head counts");
  RH_REQUIRE(head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128,
             "decode attention: head_dim must be 16, 32, 64 or 128");
  RH_REQUIRE(block_size > 0, "decode attention: bad block size");
  const int chunk = rh_decode_chunk_keys(head_dim);
  RH_REQUIRE(slice_keys >= chunk && slice_keys % chunk == 0,
             "decode attention: slice_keys must be a positive multiple of rh_decode_chunk_keys(head_dim)");
  RH_REQUIRE(max_parts >= 1, "decode attention: max_parts < 1");
  RH_REQUIRE(q_row_stride % 8 == 0 && out_row_stride >= heads * head_dim,
             "decode attention: q rows must be 16-byte aligned and out rows hold heads * head_dim");
  RH_REQUIRE((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(kpool) |
              reinterpret_cast<uintptr_t>(vpool) | reinterpret_cast<uintptr_t>(dec_meta)) % 16 == 0,
             "decode attention: q, the pools and dec_meta must be 16-byte aligned");
  DecodeArgs a;
  a.q = static_cast<const half_t*>(q);
  a.q_stride = q_row_stride;
  a.kpool = static_cast<const half_t*>(kpool);
  a.vpool = static_cast<const half_t*>(vpool);
  a.dec_meta = reinterpret_cast<const int4*>(dec_meta);
  a.tables = tables;
  a.heads = heads;
  a.kv_heads = kv_heads;
  a.group = heads / kv_heads;
  a.hchunks = (a.group + 15) / 16;
  a.block_size = block_size;
  a.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz(block_size) : -1;
  a.slice = slice_keys;
  a.max_parts = max_parts;
  a.groups_total = n_dec * kv_heads * a.hchunks;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.part_o = part_o;
  a.part_ml = part_ml;
  a.counters = counters;
  a.out = static_cast<half_t*>(out);
  a.out_stride = out_row_stride;
  const int grid = (a.groups_total + 7) / 8 * 8 * max_parts;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // 8 waves when every wave gets at least one stage of a slice (D <= 64, two workgroups per
  // CU) or two (D = 128, one per CU), else 4. Measured at config 2: 512-key slices 18.6 ->
  // 18.3 us, 256-key slices 23.4 -> 19.6 us against 4 waves; at D = 128, 8 waves with one
  // stage each run their workgroups in two rounds.
  // A grid of at most 256 workgroups (one round on the CUs: a latency-bound launch) takes 8
  // waves from 4 stages per slice on (1 x 2048 keys: 8.57 -> 8.12 us at D64, 11.65 -> 10.41
  // at D128; slices of 2 stages stay on 4 waves: 6.16 against 6.32 us at 1 x 640).
  const int stages = slice_keys / chunk;
  const bool eight = stages >= (head_dim <= 64 ? 8 : 16) || (stages >= 4 && grid <= 256);
  switch (head_dim) {
    case 16: return launch_waves<32, 16>(a, grid, eight, s);
    case 32: return launch_waves<32, 32>(a, grid, eight, s);
    case 64: return launch_waves<64, 64>(a, grid, eight, s);
    default: return launch_waves<128, 128>(a, grid, eight, s);
  }
}

// ---- the variant that allocates nothing ------------------------------------------------
//
// Slice partials and arrival counters in one file-scope device array instead of caller
// buffers. Layout (floats/ints of 4 bytes): [kNoAllocCounters counters][part_ml][part_o];
// the counters keep a fixed place so that they stay zero between calls of any shape.
namespace relay_hip {
namespace {

constexpr size_t kNoAllocBytes = size_t(16) << 20;     // 16 MiB per device
constexpr int kNoAllocCounters = 16384;                // (token, kv head, head chunk) groups
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

__global__ void zero_words_kernel(int* p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0;
}

std::mutex g_noalloc_mu;
void* g_noalloc_ptr[kMaxDevices] = {};
hipStream_t g_noalloc_stream[kMaxDevices] = {};  // the stream of the device's last call
bool g_noalloc_used[kMaxDevices] = {};

// The device address of `scratch` on the current device, looked up (and its counters
// cleared, by a kernel so that the call may sit inside a captured graph) on the first call
// on each device.
int noalloc_scratch(hipStream_t s, void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error(std::string("decode attention (no-alloc): hipGetDevice: ") + hipGetErrorString(e));
    return static_cast<int>(e);
  }
  RH_REQUIRE(dev >= 0 && dev < kMaxDevices, "decode attention (no-alloc): device index out of range");
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  // Overlap guard: a call on another stream than the device's previous call is refused while
  // that stream still has work queued (the previous call's kernel may still be using the
  // array). Calls on one stream are ordered by the stream and need no check. A stream under
  // graph capture cannot be queried; such calls (and replays of captured graphs) are not
  // checked.
  if (g_noalloc_used[dev] && g_noalloc_stream[dev] != s) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cap) == hipSuccess && cap == hipStreamCaptureStatusNone &&
        hipStreamQuery(g_noalloc_stream[dev]) == hipErrorNotReady) {
      (void)hipGetLastError();
      set_error("decode attention (no-alloc): the previous call on this GPU, on another stream, may still be running; "
                "calls of the no-alloc entry point share one scratch array per GPU and must not overlap");
      return -1;
    }
    (void)hipGetLastError();  // a query of a stream that no longer exists leaves an error behind
  }
  if (!g_noalloc_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_error(std::string("decode attention (no-alloc): hipGetSymbolAddress: ") + hipGetErrorString(e));
      return e != hipSuccess ? static_cast<int>(e) : -1;
    }
    RH_TRY_LAUNCH(hipLaunchKernelGGL(zero_words_kernel, dim3(64), dim3(256), 0, s, static_cast<int*>(p),
                                     kNoAllocCounters));
    g_noalloc_ptr[dev] = p;
  }
  *out = g_noalloc_ptr[dev];
  g_noalloc_stream[dev] = s;
  g_noalloc_used[dev] = true;
  return 0;
}

}  // namespace
}  // namespace relay_hip

extern "C" size_t rh_decode_noalloc_scratch_bytes(void) { return kNoAllocBytes; }

extern "C" int rh_paged_decode_attention_noalloc(const void* q, int64_t q_row_stride, const void* kpool,
                                                 const void* vpool, const int* dec_meta, const int* tables, int n_dec,
                                                 int heads, int kv_heads, int head_dim, int block_size, int slice_keys,
                                                 int max_parts, float scale, void* out, int64_t out_row_stride,
                                                 void* stream) {
  if (n_dec == 0) return 0;
  RH_REQUIRE(n_dec > 0 && heads > 0 && kv_heads > 0 && heads % kv_heads == 0 && max_parts >= 1,
             "decode attention (no-alloc): bad sizes");
  const size_t groups = static_cast<size_t>(n_dec) * kv_heads * ((heads / kv_heads + 15) / 16);
  const size_t partials = static_cast<size_t>(n_dec) * heads * max_parts;
  const size_t words = kNoAllocCounters + partials * 2 + partials * static_cast<size_t>(head_dim);
  RH_REQUIRE(groups <= static_cast<size_t>(kNoAllocCounters) && words * 4 <= kNoAllocBytes,
             "decode attention (no-alloc): n_dec * heads * max_parts * (head_dim + 2) exceeds the static scratch "
             "(rh_decode_noalloc_scratch_bytes); use rh_paged_decode_attention with caller buffers");
  hipStream_t s = static_cast<hipStream_t>(stream);
  void* base = nullptr;
  if (int rc = noalloc_scratch(s, &base)) return rc;
  int* counters = static_cast<int*>(base);
  float* part_ml = reinterpret_cast<float*>(counters + kNoAllocCounters);
  float* part_o = part_ml + partials * 2;
  return rh_paged_decode_attention(q, q_row_stride, kpool, vpool, dec_meta, tables, n_dec, heads, kv_heads, head_dim,
                                   block_size, slice_keys, max_parts, scale, part_o, part_ml, counters, out,
                                   out_row_stride, stream);
}
