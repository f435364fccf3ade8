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
// coordinate. A codebook that is not strictly increasing, with two switch
// points in one cell, or with a switch point below 2^-60 in magnitude, falls
// back to the scan.
//
// Direction on the table path: dir = q0 + e * inv with inv = RN(1 / r) (one
// correctly rounded division per vector), q0 = RN(y * inv) and the residual
// e = fma(-r, q0, y). By Markstein's theorem this is RN(y / r), the
// reference's division, whenever e is exact, which holds when
// exp(r) + exp(q0) - 46 >= -149. The fast form is taken per 16-vector tile
// when every radius is finite and >= 2^-40 (or zero-like, dir = 0): then every
// direction within a factor of two of a switch point (>= 2^-60) is exact, and a
// direction off by an ulp elsewhere crosses no switch point, so the index is
// the reference's. Tiles with other radii divide per coordinate.
#include "pqkv_device.h"
#include "pqkv_launch.h"

namespace pqkv {

namespace {

constexpr int kEW = 4;              // waves per workgroup
constexpr int kECells = 1024;       // direction cells over [-1, 1], 1/512 wide
constexpr int kECellSlots = kECells + 3;  // cell u covers [u - 513, u - 512) / 512
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

// The same scan as a rolled loop over the LDS codebook: the fallback path's
// form, which keeps the codebook out of registers.
__device__ __forceinline__ int scan_index_rolled(float d, const float *cb, int nl) {
#pragma clang fp contract(off)
  int b = 0;
  float m = 1e30f;
#pragma nounroll
  for (int i = 0; i < nl; ++i) {
    const float e = fabsf(d - cb[i]);
    if (e < m) {
      m = e;
      b = i;
    }
  }
  return b;
}

// Direction cell, monotone in d (the table is built with the same function;
// a rounded fma of a monotone exact function is monotone). For |d| <= 1 + 2^-9
// the clamp never acts: dir_cell_unclamped is the same function there.
__device__ __forceinline__ int dir_cell_unclamped(float d) {
  return (int)__builtin_fmaf(d, (float)(kECells / 2), (float)(kECells / 2 + 1));
}
__device__ __forceinline__ int dir_cell(float d) {
  return min(max(dir_cell_unclamped(d), 0), kECellSlots - 1);
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

template <bool B>
struct TableFlag {
  static constexpr bool on = B;
};

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
__global__ void __launch_bounds__(kEW * 64, 2) encode_mfma_kernel(const EncodeArgs a, float *rot_out,
                                                                            float *radius_out) {
  constexpr int MT = D / 16;            // output-coordinate tiles
  constexpr int KS = D / 32;            // k-steps over input coordinates
  constexpr int NL = 1 << BITS;
  constexpr int VB = vector_bytes(D, BITS);
  constexpr int SEGS = MT * KS * 2 * 2; // (mt, ks, plane, half)
  __shared__ __attribute__((aligned(16))) uint8_t rl[SEGS * kESeg];
  __shared__ uint2 cells[kECellSlots];  // (index at the cell start, switch point bits or +inf)
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
  // ---- switch points: 16 lanes per point i search (c_i, c_{i+1}] 16-ary:
  // lane j tests the (j + 1)/16 point of the range, the first that the scan
  // maps to i + 1 or more closes it. Keys of fp32 values differ by < 2^33,
  // so 9 steps reach a range of one. ----
  {
    const int i = tid >> 4, j = tid & 15;
    const bool act = i < NL - 1;
    bool ok = act;
    int64_t lo = 0, hi = 0;
    if (act) {
      ok = cb[i] < cb[i + 1] && scan_index(cb[i], cb, NL) <= i && scan_index(cb[i + 1], cb, NL) >= i + 1;
      lo = fkey(cb[i]);
      hi = fkey(cb[i + 1]);
    }
    for (int step = 0; step < 10; ++step) {
      const int64_t span = hi - lo;
      const int64_t cand = j == 15 ? hi : lo + ((span * (j + 1)) >> 4);
      const bool p = ok && span > 1 && scan_index(kfloat(cand), cb, NL) >= i + 1;
      const uint32_t gm = (uint32_t)(__builtin_amdgcn_ballot_w64(p) >> (16 * (i & 3))) & 0xFFFFu;
      const int k = gm ? __builtin_ctz(gm) : 15;
      if (ok && span > 1) {
        const int64_t nhi = k == 15 ? hi : lo + ((span * (k + 1)) >> 4);
        lo = k == 0 ? lo : lo + ((span * k) >> 4);
        hi = nhi;
      }
    }
    if (act && j == 0) {
      if (!ok || hi - lo != 1) {
        table_ok = 0;
      } else {
        thr[i] = kfloat(hi);
        ucell[i] = dir_cell(kfloat(hi));
        if (!(fabsf(thr[i]) >= 0x1p-60f)) table_ok = 0;
      }
    }
  }
  __syncthreads();
  for (int u = tid; u < kECellSlots; u += kEW * 64) {
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

  const half_t *x = (const half_t *)a.x;
  // vector v = n_inner * vo + vi; the host keeps n below 2^32
  const uint32_t n = (uint32_t)(a.n_outer * a.n_inner);
  const int64_t groups = ((int64_t)n + kEVec - 1) / kEVec;
  const FastDiv by_inner((uint32_t)a.n_inner);
  const bool rows = a.n_outer > 1;
  auto split = [&](uint32_t v, uint32_t &vo, uint32_t &vi) {
    vo = rows ? by_inner.div(v) : 0u;
    vi = v - vo * (uint32_t)a.n_inner;
  };
  // The table test is uniform per workgroup: one copy of the loop per path,
  // so no branch sits between the per-coordinate table reads.
  // B operand: lane (col, grp), tile c holds vector 64 g + 16 c + col, input
  // coordinates 32 ks + 8 grp .. + 7 (zeros past the end).
  auto load_x = [&](int64_t g, half8_t (&xb)[4][KS]) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t v = (uint32_t)g * kEVec + 16 * c + col;
      uint32_t vo, vi;
      split(v, vo, vi);
      const half_t *xv = x + (int64_t)vo * a.x_outer_stride + (int64_t)vi * D;
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
  };
  const int64_t g_step = (int64_t)gridDim.x * kEW;
  auto run = [&](auto flag) {
  constexpr bool kTable = decltype(flag)::on;
  half8_t xb[4][KS];
  int64_t g = (int64_t)blockIdx.x * kEW + wave;
  if (g < groups) load_x(g, xb);
  for (; g < groups; g += g_step) {
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
    // The next group's input streams in while this one is quantised.
    if (g + g_step < groups) load_x(g + g_step, xb);

    // ---- per vector: radius tree, direction, index, packing ----
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float y[MT][4];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) y[mt][i] = acc[c][mt][i];
      int64_t vo_bytes;
      {
        const uint32_t v = (uint32_t)g * kEVec + 16 * c + col;
        uint32_t vo, vi;
        split(v, vo, vi);
        vo_bytes = v < n ? (int64_t)vo * a.blocks_outer_stride + (int64_t)vi * VB : -1;
      }
      if (rot_out != nullptr && vo_bytes >= 0) {
        const int64_t v = (int64_t)g * kEVec + 16 * c + col;
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
      if (radius_out != nullptr && vo_bytes >= 0 && grp == 0) radius_out[(int64_t)g * kEVec + 16 * c + col] = r;
      const bool nz = r > 1e-30f;
      int code[MT][4];
      if constexpr (kTable) {
        // Fast form for the tile when every radius is zero-like (dir = 0,
        // reached through inv = 0 on finite y) or finite and >= 2^-40
        // (Markstein quotient exact, |dir| <= 1 + 11 ulp so the cell needs no
        // clamp). A NaN radius (dir = 0 by the reference, but y * 0 is NaN)
        // takes the per-coordinate form.
        const bool fast = r <= 1e-30f || (r >= 0x1p-40f && r < __builtin_inff());
        if (__builtin_amdgcn_ballot_w64(!fast) == 0) {
          const float inv = nz ? __fdiv_rn(1.0f, r) : 0.0f;
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              float d;
              {
#pragma clang fp contract(off)
                const float q0 = y[mt][i] * inv;
                const float e = __builtin_fmaf(-r, q0, y[mt][i]);
                d = __builtin_fmaf(e, inv, q0);
              }
              const uint2 ce = cells[dir_cell_unclamped(d)];
              code[mt][i] = (int)ce.x + (d >= __builtin_bit_cast(float, ce.y) ? 1 : 0);
            }
        } else {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              float d = nz ? __fdiv_rn(y[mt][i], r) : 0.0f;
              d = d == d ? d : -2.0f;  // NaN: index 0, as the scan gives
              const uint2 ce = cells[dir_cell(d)];
              code[mt][i] = (int)ce.x + (d >= __builtin_bit_cast(float, ce.y) ? 1 : 0);
            }
        }
      } else {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float d = nz ? __fdiv_rn(y[mt][i], r) : 0.0f;
            code[mt][i] = scan_index_rolled(d, cb, NL);
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
          if (grp < D / 32) *(uint16_t *)(out + grp * kPq4BlockBytes) = radius_half_bits(r);
        } else {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const uint32_t b1 = (uint32_t)(code[mt][0] | (code[mt][1] << 2) | (code[mt][2] << 4) | (code[mt][3] << 6));
            out[(mt >> 1) * kPq2BlockBytes + 2 + 4 * (mt & 1) + grp] = (uint8_t)b1;
          }
          if (grp < D / 32) *(uint16_t *)(out + grp * kPq2BlockBytes) = radius_half_bits(r);
        }
      }
    }
  }
  };
  if (table_ok != 0) run(TableFlag<true>{});
  else run(TableFlag<false>{});
}

hipError_t launch_encode_mfma(const EncodeArgs &a, float *rot_out, float *radius_out, int cus, hipStream_t s) {
  const int64_t n = a.n_outer * a.n_inner;
  const int64_t groups = (n + kEVec - 1) / kEVec;
  // each workgroup builds its R operand and centroid table once, so one
  // resident round (the launch bounds give two per CU) loops over the groups
  int64_t grid = (groups + kEW - 1) / kEW;
  if (grid > 2 * (int64_t)cus) grid = 2 * (int64_t)cus;
  if (grid < 1) grid = 1;
#define PQKV_EM(DD, BB) encode_mfma_kernel<DD, BB><<<(int)grid, kEW * 64, 0, s>>>(a, rot_out, radius_out)
  if (a.d == 128 && a.bits == 4) PQKV_EM(128, 4);
  else if (a.d == 128 && a.bits == 2) PQKV_EM(128, 2);
  else if (a.d == 64 && a.bits == 4) PQKV_EM(64, 4);
  else PQKV_EM(64, 2);
#undef PQKV_EM
  return hipGetLastError();
}

}  // namespace pqkv
