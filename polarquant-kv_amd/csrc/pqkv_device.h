// Device-side helpers shared by the gfx950 kernels of libpqkv_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pqkv_layout.h"

namespace pqkv {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// bfloat16 storage: the upper half of an fp32, so widening is exact.
struct bf16_t {
  uint16_t bits;
};
__device__ __forceinline__ float bf16_to_float(uint32_t bits16) { return __builtin_bit_cast(float, bits16 << 16); }

constexpr int kWave = 64;

__device__ __forceinline__ float half_bits_to_float(uint32_t bits16) {
  uint16_t b = (uint16_t)bits16;
  half_t h = __builtin_bit_cast(half_t, b);
  return (float)h;
}

__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
  half_t h = (half_t)f;   // v_cvt_f16_f32: round to nearest even
  return __builtin_bit_cast(uint16_t, h);
}

// The stored block radius: fp16 (RNE) of r saturated to the largest finite
// fp16, 65504, as the reference stores fp16 radii
// (src/polarquant_kv_cuda/compress_kernel.py:178, clamp(-65504, 65504).half()).
// A NaN radius stays NaN.
__device__ __forceinline__ uint16_t radius_half_bits(float r) {
  return float_to_half_bits(r > 65504.0f ? 65504.0f : r);
}

// Unsigned division by a divisor fixed per launch (Granlund and Montgomery,
// "Division by invariant integers using multiplication", 1994, round-up
// multiplier with the add-back step): exact for every 32-bit numerator.
struct FastDiv {
  uint32_t d, m;
  int s1, s2;
  __device__ explicit FastDiv(uint32_t div) : d(div) {
    int l = 0;
    while (l < 32 && (1ull << l) < div) ++l;
    m = (uint32_t)((((uint64_t)1 << 32) * (((uint64_t)1 << l) - div)) / div + 1);
    s1 = l < 1 ? l : 1;
    s2 = l > 1 ? l - 1 : 0;
  }
  __device__ __forceinline__ uint32_t div(uint32_t n) const {
    const uint32_t t = __umulhi(m, n);
    return (t + ((n - t) >> s1)) >> s2;
  }
};

__device__ __forceinline__ float shfl_down_f(float v, int s) { return __shfl_down(v, s, kWave); }
__device__ __forceinline__ float shfl_xor_f(float v, int s) { return __shfl_xor(v, s, kWave); }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int s = 32; s > 0; s >>= 1) v = fmaxf(v, shfl_xor_f(v, s));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int s = 32; s > 0; s >>= 1) v += shfl_xor_f(v, s);
  return v;
}

// v_alignbyte_b32: bytes [sh .. sh+3] of the 64-bit value hi:lo.
__device__ __forceinline__ uint32_t align_bytes(uint32_t hi, uint32_t lo, uint32_t sh) {
  return __builtin_amdgcn_alignbyte(hi, lo, sh);
}

__device__ __forceinline__ float fdot2(half2_t a, half2_t b, float c) {
  return __builtin_amdgcn_fdot2(a, b, c, false);
}

}  // namespace pqkv
