// Fast fused encoder on the matrix cores (gfx950) for fp16 input vectors:
// rotate, radius, direction, nearest centroid, block_pq4 / block_pq2 packing.
//
// Rotation: Y^T = R . X^T with v_mfma_f32_16x16x32_f16. A = R (16 output
// coordinates x 32 input coordinates, from LDS), B = X^T (the fp16 input, 16
// vectors per tile, straight from HBM). fp16 input is exact, so only R is
// split (R = R_hi + R_lo, R_lo = fp16(R - R_hi), subnormals kept by the MFMA):
// two MFMAs per tile product give fp32-grade rotated values (not the FMA-chain
// rounding of the exact encoder; the quantiser below is bit-exact on the
// values this rotation produces).
//
// The result lands with lane (col, grp) holding output coordinates
// 16 mt + 4 grp + i of vector col, which maps the reference's 128-slot tree of
// squares (slot t += slot t + s for s = 64 .. 1) onto the lanes exactly: s = 64,
// 32, 16 are in-lane (mt + 4, + 2, + 1), s = 8 and 4 are the permlane32 / 16
// swaps (lanes + 32, + 16; both sides add the same pair, and IEEE addition
// commutes), s = 2, 1 are in-lane (i + 2, i + 1).
//
// Nearest centroid: the reference scans |dir - c_i| and keeps the first
// minimum. For a sorted codebook that index is a step function of dir, so it
// equals the number of switch points theta_i <= dir, where theta_i is the
// smallest fp32 value the scan maps to i + 1. Each workgroup finds the
// switch points by bisection over fp32 values with the scan itself, then
// builds a table over 1024 direction cells holding (index at the cell start,
// the switch point inside the cell): one LDS read and one compare per
// coordinate. A codebook that is not strictly increasing, or with two switch
// points in one cell, falls back to the scan.
#include "pqkv_device.h"
#include "pqkv_launch.h"

namespace pqkv {

namespace {

constexpr int kEW = 4;              // waves per workgroup
constexpr int kECells = 1024;       // direction cells over [-1, 1]
constexpr int kESeg = 64 * 8;       // one operand segment: 64 lanes x 8 bytes
constexpr int kEVec = 64;           // vectors per wave iteration (4 tiles of 16)

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) u32x2 lds_u32x2;
typedef __attribute__((address_space(3))) const u32x2 lds_cu32x2;

__device__ __forceinline__ void lds_put8(uint8_t *p, uint32_t a, uint32_t b) { *(lds_u32x2 *)p = (u32x2){a, b}; }
__device__ __forceinline__ u32x2 lds_get8(const uint8_t *p) { return *(lds_cu32x2 *)p; }

__device__ __forceinline__ half8_t pack8u(u32x2 a, u32x2 b) {
  typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
  u32x4v v = {a.x, a.y, b.x, b.y};
  return __builtin_bit_cast(half8_t, v);
}

__device__ __forceinline__ float4_t mfma16(half8_t a, half8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t pack_h2(half_t a, half_t b) {
  half2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float swap32_add(float x) {
  auto s = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x), false, false);
  return __builtin_bit_cast(float, (uint32_t)s[0]) + __builtin_bit_cast(float, (uint32_t)s[1]);
}
__device__ __forceinline__ float swap16_add(float x) {
  auto s = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x), false, false);
  return __builtin_bit_cast(float, (uint32_t)s[0]) + __builtin_bit_cast(float, (uint32_t)s[1]);
}

// The reference quantiser: first i minimising |d - c_i| (strict '<').
__device__ __forceinline__ int scan_index(float d, const float *cb, int nl) {
#pragma clang fp contract(off)
  int b = 0;
  float m = 1e30f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    if (i < nl) {
      const float e = fabsf(d - cb[i]);
      if (e < m) {
        m = e;
        b = i;
      }
    }
  }
  return b;
}

// Direction cell, monotone in d (the table is built with the same function).
__device__ __forceinline__ int dir_cell(float d) {
#pragma clang fp contract(off)
  const float t = (d + 1.0f) * (float)(kECells / 2);
  const int u = (int)t;
  return min(max(u, 0), kECells);
}

// Order-preserving map between fp32 values and integers.
__device__ __forceinline__ int64_t fkey(float f) {
  const int32_t i = __builtin_bit_cast(int32_t, f);
  return i >= 0 ? (int64_t)i : -(int64_t)(i & 0x7FFFFFFF);
}
__device__ __forceinline__ float kfloat(int64_t k) {
  return k >= 0 ? __builtin_bit_cast(float, (int32_t)k) : __builtin_bit_cast(float, (int32_t)(0x80000000u | (uint32_t)(-k)));
}

}  // namespace

template <int D, int BITS>
__global__ void __launch_bounds__(kEW * 64, 2) encode_mfma_kernel(const EncodeArgs a, float *rot_out) {
  constexpr int MT = D / 16;            // output-coordinate tiles
  constexpr int KS = D / 32;            // k-steps over input coordinates
  constexpr int NL = 1 << BITS;
  constexpr int VB = vector_bytes(D, BITS);
  constexpr int SEGS = MT * KS * 2 * 2; // (mt, ks, plane, half)
  __shared__ __attribute__((aligned(16))) uint8_t rl[SEGS * kESeg];
  __shared__ uint2 cells[kECells + 1];  // (index at the cell start, switch point bits or +inf)
  __shared__ float cb[16], thr[16];
  __shared__ int ucell[16];
  __shared__ int table_ok;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;

  // ---- R as the A operand: seg(mt, ks, plane, h), lane 16 grp + col holds
  // R[16 mt + col][32 ks + 8 grp + 4 h .. + 3] ----
  for (int it = tid; it < D * D / 4; it += kEW * 64) {
    const int j = it / (D / 4), q = it % (D / 4);
    const float4 r4 = *(const float4 *)(a.R + (int64_t)j * D + 4 * q);
    const float rv[4] = {r4.x, r4.y, r4.z, r4.w};
    half_t hi[4], lo[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      hi[u] = (half_t)rv[u];
      lo[u] = (half_t)(rv[u] - (float)hi[u]);
    }
    const int mt = j >> 4, c = j & 15, ks = q >> 3, g = (q >> 1) & 3, h = q & 1;
    const int seg = ((mt * KS + ks) * 2 + 0) * 2 + h;
    uint8_t *p = rl + seg * kESeg + (16 * g + c) * 8;
    lds_put8(p, pack_h2(hi[0], hi[1]), pack_h2(hi[2], hi[3]));
    lds_put8(p + 2 * kESeg, pack_h2(lo[0], lo[1]), pack_h2(lo[2], lo[3]));  // plane 1 is two segments on
  }
  if (tid < 16) cb[tid] = tid < NL ? a.codebook[tid] : 0.0f;
  if (tid == 0) table_ok = 1;
  __syncthreads();
  // ---- switch points: lane i of wave 0 bisects between c_i and c_{i+1} ----
  if (tid < NL - 1) {
    const int i = tid;
    if (!(cb[i] < cb[i + 1])) {
      table_ok = 0;
    } else {
      int64_t lo = fkey(cb[i]), hi = fkey(cb[i + 1]);
      if (scan_index(cb[i], cb, NL) > i || scan_index(cb[i + 1], cb, NL) < i + 1) table_ok = 0;
      while (hi - lo > 1) {
        const int64_t mid = lo + (hi - lo) / 2;
        if (scan_index(kfloat(mid), cb, NL) >= i + 1) hi = mid;
        else lo = mid;
      }
      thr[i] = kfloat(hi);
      ucell[i] = dir_cell(kfloat(hi));
    }
  }
  __syncthreads();
  for (int u = tid; u <= kECells; u += kEW * 64) {
    int base = 0, inside = -1, count = 0;
    for (int i = 0; i < NL - 1; ++i) {
      if (ucell[i] < u) ++base;
      else if (ucell[i] == u) {
        inside = i;
        ++count;
      }
    }
    if (count > 1) table_ok = 0;
    cells[u] = make_uint2((uint32_t)base, inside >= 0 ? __builtin_bit_cast(uint32_t, thr[inside]) : 0x7F800000u);
  }
  __syncthreads();
  const bool use_table = table_ok != 0;

  const half_t *x = (const half_t *)a.x;
  const int64_t n = a.n_outer * a.n_inner;
  const int64_t groups = (n + kEVec - 1) / kEVec;
  for (int64_t g = (int64_t)blockIdx.x * kEW + wave; g < groups; g += (int64_t)gridDim.x * kEW) {
    // ---- B operand: lane (col, grp), tile c holds vector 64 g + 16 c + col,
    // input coordinates 32 ks + 8 grp .. + 7 ----
    half8_t xb[4][KS];
    int64_t vout[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int64_t v = g * kEVec + 16 * c + col;
      int64_t vo = 0, vi = v;
      if (a.n_outer > 1) {
        vo = v / a.n_inner;
        vi = v - vo * a.n_inner;
      }
      vout[c] = v < n ? vo * a.blocks_outer_stride + vi * VB : -1;
      const half_t *xv = x + vo * a.x_outer_stride + vi * D;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if (v < n) {
          xb[c][ks] = *(const half8_t *)(xv + 32 * ks + 8 * grp);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) xb[c][ks][e] = (half_t)0.0f;
        }
      }
    }
    float4_t acc[4][MT];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[c][mt] = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const uint8_t *s0 = rl + ((mt * KS + ks) * 2 * 2) * kESeg + lane * 8;
        const half8_t ah = pack8u(lds_get8(s0), lds_get8(s0 + kESeg));
        const half8_t al = pack8u(lds_get8(s0 + 2 * kESeg), lds_get8(s0 + 3 * kESeg));
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          acc[c][mt] = mfma16(ah, xb[c][ks], acc[c][mt]);
          acc[c][mt] = mfma16(al, xb[c][ks], acc[c][mt]);
        }
      }

    // ---- per vector: radius tree, direction, index, packing ----
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float y[MT][4];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) y[mt][i] = acc[c][mt][i];
      const int64_t vo_bytes = vout[c];
      if (rot_out != nullptr && vo_bytes >= 0) {
        const int64_t v = g * kEVec + 16 * c + col;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i) rot_out[v * D + 16 * mt + 4 * grp + i] = y[mt][i];
      }
      float r;
      {
#pragma clang fp contract(off)
        float t[MT][4];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i) t[mt][i] = y[mt][i] * y[mt][i];
        // slots 16 mt + 4 grp + i; the s = 64 step exists for D = 128 only
        float v0[4], v1[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float s0 = t[0][i], s1 = t[1][i], s2 = t[2][i], s3 = t[3][i];
          if (D == 128) {
            s0 = s0 + t[4][i];
            s1 = s1 + t[5][i];
            s2 = s2 + t[6][i];
            s3 = s3 + t[7][i];
          }
          s0 = s0 + s2;                 // s = 32
          s1 = s1 + s3;
          v0[i] = s0 + s1;              // s = 16
          v0[i] = swap32_add(v0[i]);    // s = 8: slots t, t + 8 (lanes +32)
          v1[i] = swap16_add(v0[i]);    // s = 4: slots t, t + 4 (lanes +16)
        }
        const float w0 = v1[0] + v1[2];  // s = 2
        const float w1 = v1[1] + v1[3];
        const float tot = w0 + w1;       // s = 1
        r = (float)__builtin_sqrt((double)tot);
      }
      const bool nz = r > 1e-30f;
      int code[MT][4];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float d = nz ? __fdiv_rn(y[mt][i], r) : 0.0f;
          if (use_table) {
            const uint2 e = cells[dir_cell(d)];
            code[mt][i] = (int)e.x + (d >= __builtin_bit_cast(float, e.y) ? 1 : 0);
          } else {
            code[mt][i] = scan_index(d, cb, NL);
          }
        }
      if (vo_bytes >= 0) {
        uint8_t *out = a.blocks + vo_bytes;
        if (BITS == 4) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const uint32_t b2 = (uint32_t)(code[mt][0] | (code[mt][1] << 4)) |
                                ((uint32_t)(code[mt][2] | (code[mt][3] << 4)) << 8);
            *(uint16_t *)(out + (mt >> 1) * kPq4BlockBytes + 2 + 8 * (mt & 1) + 2 * grp) = (uint16_t)b2;
          }
          if (grp < D / 32) *(uint16_t *)(out + grp * kPq4BlockBytes) = float_to_half_bits(r);
        } else {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const uint32_t b1 = (uint32_t)(code[mt][0] | (code[mt][1] << 2) | (code[mt][2] << 4) | (code[mt][3] << 6));
            out[(mt >> 1) * kPq2BlockBytes + 2 + 4 * (mt & 1) + grp] = (uint8_t)b1;
          }
          if (grp < D / 32) *(uint16_t *)(out + grp * kPq2BlockBytes) = float_to_half_bits(r);
        }
      }
    }
  }
}

hipError_t launch_encode_mfma(const EncodeArgs &a, float *rot_out, hipStream_t s) {
  const int64_t n = a.n_outer * a.n_inner;
  const int64_t groups = (n + kEVec - 1) / kEVec;
  int64_t grid = (groups + kEW - 1) / kEW;
  if (grid > 1024) grid = 1024;
  if (grid < 1) grid = 1;
#define PQKV_EM(DD, BB) encode_mfma_kernel<DD, BB><<<(int)grid, kEW * 64, 0, s>>>(a, rot_out)
  if (a.d == 128 && a.bits == 4) PQKV_EM(128, 4);
  else if (a.d == 128 && a.bits == 2) PQKV_EM(128, 2);
  else if (a.d == 64 && a.bits == 4) PQKV_EM(64, 4);
  else PQKV_EM(64, 2);
#undef PQKV_EM
  return hipGetLastError();
}

}  // namespace pqkv
