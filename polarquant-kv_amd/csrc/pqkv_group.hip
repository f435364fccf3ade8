// Group (min / scale) quantisation of rotated directions: the reference's
// CPU format (python/polarquant_kv/quantizer.py:25-158) on the GPU.
//
// compress, per vector v (fp32 or fp16, d <= 256):
//   y = fp32(fp64(v) R^T)          (rotation.py:48: fp64 product, cast back)
//   r = |y| (fp32)                  (quantizer.py:105)
//   r < 1e-30: r = 0, codes 0, mins 0, scales 1   (quantizer.py:107-118)
//   u = y / r (fp32), zero-padded to d_pad = ceil(d / gs) gs
//   per group of gs values: lo = min, hi = max, s = (hi - lo) / levels if
//   hi > lo else 1; code = clip(rint((u - lo) / s), 0, levels), 0 for a flat
//   group (quantizer.py:25-66), levels = 2^bits - 1
// decompress: u = code * s + lo (fp32, two roundings), y = u[:d] r,
// v = fp32(fp64(y) R) (quantizer.py:69-85,137-158); zeros for r < 1e-30.
//
// One wave per vector: lane L owns coordinates L, L + 64, ... The rotation
// sums in fp64 in coordinate order; the reference's fp64 product rounded to
// fp32 agrees except where the fp64 sum lands within ~1e-16 of an fp32
// rounding boundary. The norm is the correctly rounded fp32 of an fp64 sum of
// squares; numpy's fp32 norm can differ from it by an ulp or two.
#include "pqkv_device.h"
#include "pqkv_launch.h"

namespace pqkv {

namespace {

constexpr int kGW = 4;          // waves (vectors in flight) per workgroup
constexpr int kGMaxD = 256;     // largest d
constexpr int kGMaxPad = 512;   // d_pad < 2 d

// Lane L's coordinates j = L + 64 i, i < kGMaxD / 64.
constexpr int kGPer = kGMaxD / 64;

}  // namespace

__global__ void __launch_bounds__(kGW * 64) group_compress_kernel(const void *x, int x_dtype, const double *R,
                                                                  int64_t n, int d, int bits, int gs, float *radius,
                                                                  uint8_t *codes, float *mins, float *scales) {
  __shared__ double xv[kGW][kGMaxD];
  __shared__ float dir[kGW][kGMaxPad];
  __shared__ float glo[kGW][kGMaxPad], gsc[kGW][kGMaxPad];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int ng = (d + gs - 1) / gs, dpad = ng * gs;
  const float levels = (float)((1 << bits) - 1);
  for (int64_t v = (int64_t)blockIdx.x * kGW + w; v < n; v += (int64_t)gridDim.x * kGW) {
    for (int j = lane; j < d; j += 64) {
      const float xf = x_dtype == PQKV_F16 ? (float)((const half_t *)x)[v * d + j] : ((const float *)x)[v * d + j];
      xv[w][j] = (double)xf;
    }
    __builtin_amdgcn_wave_barrier();
    float y[kGPer];
    double sq = 0.0;
#pragma unroll
    for (int i = 0; i < kGPer; ++i) {
      const int j = lane + 64 * i;
      y[i] = 0.0f;
      if (j < d) {
        const double *rr = R + (int64_t)j * d;
        double acc = 0.0;
        for (int k = 0; k < d; ++k) acc = __builtin_fma(xv[w][k], rr[k], acc);
        y[i] = (float)acc;
        sq += (double)y[i] * (double)y[i];
      }
    }
    // fp64 sum of the squares over the wave
    for (int s = 32; s > 0; s >>= 1) sq += __shfl_xor(sq, s, 64);
    const float r = (float)__builtin_sqrt(sq);
    const bool zero = !(r >= 1e-30f);
    float *mv = mins + v * ng;
    float *sv = scales + v * ng;
    uint8_t *cv = codes + v * dpad;
    if (zero) {
      for (int j = lane; j < dpad; j += 64) cv[j] = 0;
      for (int g = lane; g < ng; g += 64) {
        mv[g] = 0.0f;
        sv[g] = 1.0f;
      }
      if (lane == 0) radius[v] = 0.0f;
      __builtin_amdgcn_wave_barrier();
      continue;
    }
#pragma unroll
    for (int i = 0; i < kGPer; ++i) {
      const int j = lane + 64 * i;
      if (j < d) dir[w][j] = __fdiv_rn(y[i], r);
    }
    for (int j = d + lane; j < dpad; j += 64) dir[w][j] = 0.0f;
    __builtin_amdgcn_wave_barrier();
    for (int g = lane; g < ng; g += 64) {
      float lo = dir[w][g * gs], hi = lo;
      for (int k = 1; k < gs; ++k) {
        const float u = dir[w][g * gs + k];
        lo = fminf(lo, u);
        hi = fmaxf(hi, u);
      }
      const float range = hi - lo;
      const float sc = range > 0.0f ? __fdiv_rn(range, levels) : 1.0f;
      glo[w][g] = lo;
      gsc[w][g] = range > 0.0f ? sc : 0.0f;  // 0 marks a flat group (codes 0)
      mv[g] = lo;
      sv[g] = sc;
    }
    __builtin_amdgcn_wave_barrier();
    for (int j = lane; j < dpad; j += 64) {
      const int g = j / gs;
      const float sc = gsc[w][g];
      float q = 0.0f;
      if (sc > 0.0f) {
#pragma clang fp contract(off)
        q = rintf(__fdiv_rn(dir[w][j] - glo[w][g], sc));
        q = fminf(fmaxf(q, 0.0f), levels);
      }
      cv[j] = (uint8_t)q;
    }
    if (lane == 0) radius[v] = r;
    __builtin_amdgcn_wave_barrier();
  }
}

__global__ void __launch_bounds__(kGW * 64) group_decompress_kernel(const float *radius, const uint8_t *codes,
                                                                    const float *mins, const float *scales,
                                                                    const double *R, int64_t n, int d, int gs,
                                                                    float *out) {
  __shared__ double yv[kGW][kGMaxD];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int ng = (d + gs - 1) / gs, dpad = ng * gs;
  for (int64_t v = (int64_t)blockIdx.x * kGW + w; v < n; v += (int64_t)gridDim.x * kGW) {
    const float r = radius[v];
    if (!(r >= 1e-30f)) {
      for (int j = lane; j < d; j += 64) out[v * d + j] = 0.0f;
      continue;
    }
    for (int j = lane; j < d; j += 64) {
      const int g = j / gs;
      float u, yf;
      {
#pragma clang fp contract(off)
        u = (float)codes[v * dpad + j] * scales[v * ng + g] + mins[v * ng + g];
        yf = u * r;
      }
      yv[w][j] = (double)yf;
    }
    __builtin_amdgcn_wave_barrier();
    for (int j = lane; j < d; j += 64) {
      double acc = 0.0;
      for (int k = 0; k < d; ++k) acc = __builtin_fma(yv[w][k], R[(int64_t)k * d + j], acc);
      out[v * d + j] = (float)acc;
    }
    __builtin_amdgcn_wave_barrier();
  }
}

hipError_t launch_group_compress(const void *x, int x_dtype, const double *R, int64_t n, int d, int bits, int gs,
                                 float *radius, uint8_t *codes, float *mins, float *scales, hipStream_t s) {
  if (d < 1 || d > kGMaxD || gs < 1 || gs > d) return hipErrorInvalidValue;
  const int64_t blocks = (n + kGW - 1) / kGW;
  const int grid = (int)(blocks < 4096 ? blocks : 4096);
  group_compress_kernel<<<grid, kGW * 64, 0, s>>>(x, x_dtype, R, n, d, bits, gs, radius, codes, mins, scales);
  return hipGetLastError();
}

hipError_t launch_group_decompress(const float *radius, const uint8_t *codes, const float *mins, const float *scales,
                                   const double *R, int64_t n, int d, int gs, float *out, hipStream_t s) {
  if (d < 1 || d > kGMaxD || gs < 1 || gs > d) return hipErrorInvalidValue;
  const int64_t blocks = (n + kGW - 1) / kGW;
  const int grid = (int)(blocks < 4096 ? blocks : 4096);
  group_decompress_kernel<<<grid, kGW * 64, 0, s>>>(radius, codes, mins, scales, R, n, d, gs, out);
  return hipGetLastError();
}

}  // namespace pqkv
