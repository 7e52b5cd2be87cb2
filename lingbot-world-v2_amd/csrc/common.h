// Device-side helpers shared by the gfx950 kernels: vector types, bf16 packing, MFMA
// wrappers, LDS access and wave-level reductions. CDNA4 only (64-wide wavefronts).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lbw {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int32_t i32x8 __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Two fp32 -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  bf16x2 v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float round_bf16(float x) {
  __bf16 b = (__bf16)x;
  return (float)b;
}

// D = A(32x16) * B(16x32) + C, bf16 inputs, fp32 accumulate. Lane l supplies A row l%32 and
// B column l%32, each with 8 consecutive k of the k-group l/32. Lane l receives D column
// l%32, rows 8*(r/4) + 4*(l/32) + (r%4) for r = 0..15.
__device__ __forceinline__ floatx16 mfma32x32x16(const u32x4& a, const u32x4& b,
                                                 const floatx16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Lane l and lane l^32 exchange through v_permlane32_swap (VALU, no LDS round trip): the swap
// of (v, v) leaves the low half's value in one result and the high half's in the other, in
// every lane.
__device__ __forceinline__ float wave_max_xor32(float v) {
  const u32x2 r = __builtin_bit_cast(
      u32x2, __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false));
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float wave_sum_xor32(float v) {
  const u32x2 r = __builtin_bit_cast(
      u32x2, __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false));
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Workgroup barrier without __syncthreads()'s memory fence, so outstanding global loads (the
// K/V prefetch) stay in flight across it. Callers wait for the loads they need themselves; the
// empty asm statements keep the compiler from moving memory accesses across the barrier.
__device__ __forceinline__ void barrier_nofence() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ float wave_reduce_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

template <typename T>
__device__ __forceinline__ T* lds_ptr(unsigned char* base, int byte_off) {
  return reinterpret_cast<T*>(base + byte_off);
}

}  // namespace lbw
