// Split-context paged decode attention for gfx950, with the log-sum-exp merge fused in.
//
// Work unit: one workgroup per (decode token, kv head, 16-head chunk of its query group,
// slice of `slice_keys` keys), the split of relay's decode_attention_kernel
// (cuda_kernels.cuh:180-339). Four waves per workgroup; each wave walks a quarter of the
// slice in steps of 32 keys:
//
//   S^T[16 keys x 16 heads] = K[16 keys x D] * Q^T[D x 16 heads]     (MFMA 16x16x32, D/32 per tile)
//   online softmax per head, in the log2 domain, per lane (lane = head column)
//   O^T[D x 16 heads] += V^T[D x 32 keys] * P^T[32 keys x 16 heads]   (MFMA 16x16x32, D/16 tiles)
//
// All query heads of the group share one read of each K and V row (the GQA property the
// reference exploits with its per-thread G-head loop; here the heads are MFMA columns, so
// the score arithmetic costs no vector-ALU time and the kernel stays bound by HBM).
// K rows go straight from global memory into MFMA A operands: lane (c, g) loads key c of
// the tile, dims [8g, 8g+8) of each 32-wide group -- a 16-byte load. P^T comes out of the
// S^T accumulators already in B-operand order (the k slots of the PV product are a
// permutation of the 32 keys, the same for A and B). V needs the transpose V^T, which goes
// through LDS: each lane writes 16-byte row chunks, then reads single halves in column
// order; chunks are XOR-swizzled by key so the 4 key groups of a read hit disjoint banks.
//
// Loads are issued a round at a time (all of a wave's K and V for ROUND steps, 32 KB per
// wave), so each CU keeps ~256 KB of HBM reads in flight.
//
// The slices of a (token, kv head) are merged by the last of its workgroups to finish
// (an atomic counter per group, release/acquire fences at agent scope): no second kernel
// launch. Slice partials are (M, L) in the log2 domain plus the unnormalized O.
// Workgroup ids are mapped so the slices of one group land on the same XCD (ids are
// dealt round-robin over the 8 XCDs), which keeps the merge's reads in one L2.
#include "../../include/relay_hip.h"
#include "common.h"

namespace relay_hip {
namespace {

constexpr int kDecWaves = 4;
constexpr int kDecThreads = kDecWaves * kWave;
constexpr int kStepKeys = 32;
constexpr int kMaxSliceKeys = 1024;

struct DecodeArgs {
  const half_t* q;
  int64_t q_stride;
  const half_t* kpool;
  const half_t* vpool;
  const int* pos;
  const int* seq;
  const int* table_off;
  const int* tables;
  const int* decode_tokens;
  int heads, kv_heads, group, hchunks, block_size, bs_shift, slice, max_parts, groups_total;
  float scale_log2;
  float* part_o;
  float* part_ml;
  int* counters;
  half_t* out;
  int64_t out_stride;
};

__device__ __forceinline__ int block_of(int p, int bs, int shift) { return shift >= 0 ? p >> shift : p / bs; }
__device__ __forceinline__ int slot_of(int p, int bs, int shift) { return shift >= 0 ? p & (bs - 1) : p % bs; }

// Swizzle of a key's 16-byte chunks in the V staging rows.
__device__ __forceinline__ int vswz(int key) { return ((key >> 2) & 3) << 1; }

template <int D, int ROUND>
__global__ __launch_bounds__(kDecThreads, 2) void paged_decode_kernel(const DecodeArgs a) {
  constexpr int CH = D / 8;                         // 16-byte chunks per row
  constexpr int KH = D / 32;                        // 32-wide dim groups (QK MFMAs per tile)
  constexpr int DT = D / 16;                        // 16-dim tiles of O^T
  constexpr int VL = kStepKeys * CH / kWave;        // V loads per lane per step
  constexpr int VKEYS = kWave / CH;                 // keys covered by one V load
  static_assert(kDecWaves * kStepKeys * D * 2 == kDecWaves * 16 * D * 4, "merge area reuses the V staging");

  __shared__ int s_tbl[kMaxSliceKeys + 2];
  __shared__ __attribute__((aligned(16))) half_t s_v[kDecWaves][kStepKeys * D];
  __shared__ float s_m[kDecWaves][16], s_l[kDecWaves][16];
  __shared__ int s_last;

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = lane & 15, g = lane >> 4;

  // Workgroup -> (group, part), slices of one group on one XCD.
  const int b = blockIdx.x;
  const int sl = b >> 3;
  const int part = sl % a.max_parts;
  const int grp = (sl / a.max_parts) * 8 + (b & 7);
  if (grp >= a.groups_total) return;
  const int per_tok = a.kv_heads * a.hchunks;
  const int di = grp / per_tok;
  const int kvh = (grp % per_tok) / a.hchunks, hc = grp % a.hchunks;
  const int t = a.decode_tokens[di];
  const int ctx = a.pos[t] + 1;
  const int nparts = (ctx + a.slice - 1) / a.slice;
  if (part >= nparts) return;
  const int begin = part * a.slice, end = min(ctx, begin + a.slice);
  const int h0 = kvh * a.group + hc * 16;
  const int nh = min(16, a.group - hc * 16);
  const int* table = a.tables + a.table_off[a.seq[t]];
  const int bs = a.block_size, sh = a.bs_shift;

  const int fb = block_of(begin, bs, sh), lb = block_of(end - 1, bs, sh);
  for (int i = threadIdx.x; i <= lb - fb; i += kDecThreads) s_tbl[i] = table[fb + i];
  __syncthreads();

  // Q^T as B operands: lane (c, g) holds head c, dims [32h + 8g, +8).
  half8 qb[KH];
#pragma unroll
  for (int h = 0; h < KH; ++h) {
    if (c < nh) {
      qb[h] = load_half8(a.q + static_cast<int64_t>(t) * a.q_stride + static_cast<int64_t>(h0 + c) * D + 32 * h + 8 * g);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) qb[h][e] = 0;
    }
  }

  const int kpw = a.slice / kDecWaves;
  const int wb = begin + w * kpw, we = min(end, wb + kpw);
  const half_t* kbase = a.kpool;
  const half_t* vbase = a.vpool;

  float m_run = -INFINITY, l_part = 0.0f;
  float4v o[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) o[i] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

  half_t* sv = s_v[w];
  for (int r0 = wb; r0 < we; r0 += kStepKeys * ROUND) {
    half8 kr[ROUND][2][KH];
    half8 vr[ROUND][VL];
    // Issue the round's loads, in the order they are consumed.
#pragma unroll
    for (int s = 0; s < ROUND; ++s) {
      const int k0 = r0 + s * kStepKeys;
      if (k0 < we) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const int j = min(k0 + 16 * tt + c, end - 1);
          const int64_t off = kv_row_offset(s_tbl[block_of(j, bs, sh) - fb], a.kv_heads, kvh, bs, slot_of(j, bs, sh), D);
#pragma unroll
          for (int h = 0; h < KH; ++h) kr[s][tt][h] = load_half8(kbase + off + 32 * h + 8 * g);
        }
#pragma unroll
        for (int i = 0; i < VL; ++i) {
          const int j = min(k0 + VKEYS * i + lane / CH, end - 1);
          const int64_t off = kv_row_offset(s_tbl[block_of(j, bs, sh) - fb], a.kv_heads, kvh, bs, slot_of(j, bs, sh), D);
          vr[s][i] = load_half8(vbase + off + 8 * (lane % CH));
        }
      }
    }
#pragma unroll
    for (int s = 0; s < ROUND; ++s) {
      const int k0 = r0 + s * kStepKeys;
      if (k0 >= we) break;
      // This step's V rows into the wave's staging area (swizzled 16-byte chunks).
#pragma unroll
      for (int i = 0; i < VL; ++i) {
        const int kl = VKEYS * i + lane / CH, cc = lane % CH;
        *reinterpret_cast<half8*>(sv + kl * D + ((cc ^ vswz(kl)) << 3)) = vr[s][i];
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

      // S^T for the two 16-key tiles.
      float4v st[2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        st[tt] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int h = 0; h < KH; ++h) st[tt] = mfma16x16x32(kr[s][tt][h], qb[h], st[tt]);
      }
      float sc[8];
      float mx = -INFINITY;
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = k0 + 16 * tt + 4 * g + r;
          const float v = key < we ? st[tt][r] * a.scale_log2 : -INFINITY;
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
        half8 vt;
        const int d = 16 * dt + c;
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          const int kl = r < 4 ? 4 * g + r : 16 + 4 * g + (r - 4);
          vt[r] = sv[kl * D + ((((d >> 3) ^ vswz(kl))) << 3) + (d & 7)];
        }
        float4v acc = o[dt];
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] *= alpha;
        o[dt] = mfma16x16x32(vt, pt, acc);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }
  const float l_tot = group4_sum(l_part);

  // Merge the four waves' partials in LDS (the V staging area, now free).
  __syncthreads();
  float* so = reinterpret_cast<float*>(&s_v[0][0]);  // [wave][head][D]
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r = 0; r < 4; ++r) so[(w * 16 + c) * D + 16 * dt + 4 * g + r] = o[dt][r];
  if (g == 0) {
    s_m[w][c] = m_run;
    s_l[w][c] = l_tot;
  }
  __syncthreads();

  const bool single = nparts == 1;
  for (int idx = threadIdx.x; idx < nh * D; idx += kDecThreads) {
    const int hh = idx / D, d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < kDecWaves; ++ww) M = fmaxf(M, s_m[ww][hh]);
    float L = 0.0f, O = 0.0f;
#pragma unroll
    for (int ww = 0; ww < kDecWaves; ++ww) {
      const float mw = s_m[ww][hh];
      if (mw != -INFINITY) {
        const float f = fast_exp2(mw - M);
        L += f * s_l[ww][hh];
        O += f * so[(ww * 16 + hh) * D + d];
      }
    }
    if (single) {
      a.out[static_cast<int64_t>(t) * a.out_stride + static_cast<int64_t>(h0 + hh) * D + d] = static_cast<half_t>(O / L);
    } else {
      const int64_t pb = (static_cast<int64_t>(di) * a.heads + h0 + hh) * a.max_parts + part;
      a.part_o[pb * D + d] = O;
      if (d == 0) {
        a.part_ml[pb * 2] = M;
        a.part_ml[pb * 2 + 1] = L;
      }
    }
  }
  if (single) return;

  // The last workgroup of this group merges every slice.
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = atomicAdd(&a.counters[grp], 1);
    const int last = prev == nparts - 1;
    if (last) atomicExch(&a.counters[grp], 0);
    s_last = last;
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  for (int idx = threadIdx.x; idx < nh * D; idx += kDecThreads) {
    const int hh = idx / D, d = idx % D;
    const int64_t base = (static_cast<int64_t>(di) * a.heads + h0 + hh) * a.max_parts;
    float M = -INFINITY;
    for (int p = 0; p < nparts; ++p) M = fmaxf(M, __builtin_nontemporal_load(&a.part_ml[(base + p) * 2]));
    float L = 0.0f, O = 0.0f;
    for (int p = 0; p < nparts; ++p) {
      const float f = fast_exp2(__builtin_nontemporal_load(&a.part_ml[(base + p) * 2]) - M);
      L += f * __builtin_nontemporal_load(&a.part_ml[(base + p) * 2 + 1]);
      O += f * __builtin_nontemporal_load(&a.part_o[(base + p) * D + d]);
    }
    a.out[static_cast<int64_t>(t) * a.out_stride + static_cast<int64_t>(h0 + hh) * D + d] = static_cast<half_t>(O / L);
  }
}

}  // namespace
}  // namespace relay_hip

using namespace relay_hip;

extern "C" int rh_paged_decode_attention(const void* q, int64_t q_row_stride, const void* kpool, const void* vpool,
                                         const int* pos, const int* seq, const int* table_off, const int* tables,
                                         const int* decode_tokens, int n_dec, int heads, int kv_heads, int head_dim,
                                         int block_size, int slice_keys, int max_parts, float scale, float* part_o,
                                         float* part_ml, int* counters, void* out, int64_t out_row_stride,
                                         void* stream) {
  if (n_dec == 0) return 0;
  RH_REQUIRE(n_dec > 0 && heads > 0 && kv_heads > 0 && heads % kv_heads == 0, "decode attention: bad head counts");
  RH_REQUIRE(head_dim == 64 || head_dim == 128, "decode attention: head_dim must be 64 or 128");
  RH_REQUIRE(block_size > 0, "decode attention: bad block size");
  RH_REQUIRE(slice_keys >= 128 && slice_keys <= kMaxSliceKeys && slice_keys % 128 == 0,
             "decode attention: slice_keys must be a multiple of 128, at most 1024");
  RH_REQUIRE(max_parts >= 1, "decode attention: max_parts < 1");
  RH_REQUIRE(q_row_stride % 8 == 0 && out_row_stride >= heads * head_dim,
             "decode attention: q rows must be 16-byte aligned and out rows hold heads * head_dim");
  RH_REQUIRE((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(kpool) |
              reinterpret_cast<uintptr_t>(vpool)) % 16 == 0,
             "decode attention: q and the pools must be 16-byte aligned");
  DecodeArgs a;
  a.q = static_cast<const half_t*>(q);
  a.q_stride = q_row_stride;
  a.kpool = static_cast<const half_t*>(kpool);
  a.vpool = static_cast<const half_t*>(vpool);
  a.pos = pos;
  a.seq = seq;
  a.table_off = table_off;
  a.tables = tables;
  a.decode_tokens = decode_tokens;
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
  if (head_dim == 64) {
    RH_TRY_LAUNCH(hipLaunchKernelGGL((paged_decode_kernel<64, 4>), dim3(grid), dim3(kDecThreads), 0, s, a));
  } else {
    RH_TRY_LAUNCH(hipLaunchKernelGGL((paged_decode_kernel<128, 2>), dim3(grid), dim3(kDecThreads), 0, s, a));
  }
  return 0;
}
