// Shared device helpers for the gfx950 (CDNA4) kernels of the speculative verify step.
//
// Everything here is wave64-specific: lane masks, cross-lane reductions and the MFMA operand
// types assume 64-lane wavefronts and the v_mfma_f32_16x16x32_bf16 instruction of gfx950.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/omniasr_mi355x.h"

namespace omni {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// ---------------------------------------------------------------------------------------------- bf16

__device__ __forceinline__ float bf16_to_f32(uint32_t h16) { return __uint_as_float(h16 << 16); }

// fp32 -> bf16, round to nearest even; NaN becomes the canonical quiet NaN 0x7FC0 (the rounding
// rule of c10::BFloat16, which ``Tensor.to(torch.bfloat16)`` / ``type_as`` use).
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// The fp32 value a bf16 store of ``f`` reads back as.
__device__ __forceinline__ float round_through_bf16(float f) {
  return __uint_as_float(f32_to_bf16_rne(f) << 16);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_rne(lo) | (f32_to_bf16_rne(hi) << 16);
}

// Element e (0..7) of 8 packed bf16 values, as fp32.
__device__ __forceinline__ float bf16x8_elem(const u32x4_t& v, int e) {
  const uint32_t w = v[e >> 1];
  return (e & 1) ? __uint_as_float(w & 0xffff0000u) : __uint_as_float(w << 16);
}

// ---------------------------------------------------------------------------------------------- lanes

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ int wave_min_int(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, kWave));
  return v;
}

__device__ __forceinline__ long long wave_max_i64(long long v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    long long w = __shfl_xor(v, o, kWave);
    v = w > v ? w : v;
  }
  return v;
}

__device__ __forceinline__ int64_t clamp64(int64_t v, int64_t lo, int64_t hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

__host__ __device__ constexpr inline int64_t ceil_div64(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace omni

// Launch-time error: the HIP error of the last launch, or OMNI_OK.
static inline int omni_launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? OMNI_OK : (int)e;
}
