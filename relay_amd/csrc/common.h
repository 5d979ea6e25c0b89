// Device-side helpers shared by relay's gfx950 kernels: fp16 vector types, the MFMA
// instructions the attention and GEMV kernels use, wave-level reductions, and the
// error plumbing of the C ABI (include/relay_hip.h).
//
// MFMA operand layouts on CDNA (wave64), as these kernels rely on them:
//   v_mfma_f32_16x16x32_f16  D[16x16] += A[16x32] * B[32x16]
//     A: lane l holds row (l % 16), 8 consecutive k slots of group (l / 16)
//     B: lane l holds column (l % 16), the same 8 k slots of group (l / 16)
//     D: lane l holds column (l % 16), rows 4 * (l / 16) + r in register r (r < 4)
//   v_mfma_f32_32x32x16_f16  D[32x32] += A[32x16] * B[16x32]
//     A: lane l holds row (l % 32), 8 k slots of group (l / 32)
//     B: lane l holds column (l % 32), the same 8 k slots of group (l / 32)
//     D: lane l holds column (l % 32), rows 8 * (r / 4) + 4 * (l / 32) + (r % 4) in
//        register r (r < 16)
// Only the row/column placement matters for correctness: the k slot a (group, register)
// pair stands for is the same for A and B, so the kernels choose which logical k (key or
// head dimension) each slot carries, as long as both operands agree.
//
// fp16 stores of a product: hipcc turns `(half)(a * b)` into v_fma_mix*_f16, which rounds the
// exact product once, to fp16 (neither __fmul_rn nor `#pragma clang fp contract(off)` stops
// it); relay's kernels and its CPU backend round the fp32 product first and then convert,
// which differs at fp16 ties. f16_of_product keeps the two roundings.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

namespace relay_hip {

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef unsigned int uint4v __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// fp16(fp32(a * b)): the empty asm makes the rounded fp32 product opaque, so the conversion
// cannot be fused into a single-rounding v_fma_mix (it emits no instruction).
// fp32(a * b), opaque to the compiler: device code compiles with fp contraction on, so an add
// after a product may otherwise be fused with it into one fma in one kernel and not in
// another. The merges of split products scale the merged sum with this, then add (the
// residual, beta y), so every kernel that merges the same partials gives the same bits.
__device__ __forceinline__ float mul_rounded(float a, float b) {
  float p = a * b;
  asm("" : "+v"(p));
  return p;
}

__device__ __forceinline__ half_t f16_of_product(float a, float b) {
  float p = a * b;
  asm("" : "+v"(p));
  return static_cast<half_t>(p);
}

// ds_read_b64_tr_b16 (gfx950), as measured on MI355X: within each group of 16 lanes, lane i
// receives element i % 4 of the 8 bytes read by lanes 4j + i / 4 of its group, j = 0..3. So
// when lane s of a group reads row (r0 + s / 4), columns c0 + 4 (s % 4) .. +3 of a row-major
// fp16 matrix, lane i receives rows r0 .. r0 + 3 of column c0 + i: the k-major MFMA operand.
__device__ __forceinline__ half4 tr_read_b64(const half_t* lds_addr) {
  typedef short short4_t __attribute__((ext_vector_type(4)));
  const short4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) short4_t*)(const_cast<half_t*>(lds_addr)));
  return __builtin_bit_cast(half4, v);
}

__device__ __forceinline__ float4v mfma16x16x32(half8 a, half8 b, float4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float16v mfma32x32x16(half8 a, half8 b, float16v c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// 16 bytes from global memory as 8 halves (a plain dwordx4 load).
__device__ __forceinline__ half8 load_half8(const half_t* p) {
  uint4v v = *reinterpret_cast<const uint4v*>(p);
  return __builtin_bit_cast(half8, v);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Sum over the 4 lanes {l, l^16, l^32, l^48} (the 4 row groups of a 16x16 MFMA tile).
__device__ __forceinline__ float group4_sum(float v) {
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

__device__ __forceinline__ float group4_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 16));
  v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}

// 2^x on the hardware exp unit (v_exp_f32); exp2(-inf) = 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Offset of (position p, kv head) in one layer's paged cache, in elements.
__device__ __forceinline__ int64_t kv_row_offset(int block, int kv_heads, int kvh, int block_size, int slot, int D) {
  return ((static_cast<int64_t>(block) * kv_heads + kvh) * block_size + slot) * static_cast<int64_t>(D);
}

// Stores and loads that are coherent across the device's XCDs for this location (sc1
// accesses): how partial results pass between workgroups (a slice or K-range merge by the
// last workgroup to arrive, ordered by an agent-scope atomic counter).
__device__ __forceinline__ void coherent_store(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float coherent_load(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace relay_hip

// ---- host-side error plumbing for the C ABI ------------------------------------------

namespace relay_hip {
void set_error(const std::string& msg);
}  // namespace relay_hip

#define RH_TRY_LAUNCH(expr)                                                                 \
  do {                                                                                      \
    expr;                                                                                   \
    hipError_t _e = hipGetLastError();                                                      \
    if (_e != hipSuccess) {                                                                 \
      relay_hip::set_error(std::string("HIP launch: ") + hipGetErrorString(_e) + " in " + __func__); \
      return static_cast<int>(_e);                                                          \
    }                                                                                       \
  } while (0)

#define RH_REQUIRE(cond, msg)             \
  do {                                    \
    if (!(cond)) {                        \
      relay_hip::set_error(msg);          \
      return -1;                          \
    }                                     \
  } while (0)
