// Nearest-centroid lookup table shared by the encoders.
//
// The reference quantiser (csrc/flash_turboquant.cu:162-170) scans
// |dir - c_i| over the codebook and keeps the first minimum. For a strictly
// increasing codebook that index is a step function of dir: it equals the
// number of switch points theta_i <= dir, where theta_i is the smallest fp32
// value the scan maps to i + 1. build_cell_table() finds the switch points
// (a probe around each midpoint, a second one half an ulp from zero for a
// pair symmetric about it, then a 16-ary search over fp32 values, all with a
// test equivalent to the scan there), then fills a table over 1027
// direction cells holding (index at the cell start, the switch point inside
// the cell or +inf): one LDS read and one compare per coordinate. The
// cell of dir is round(512 dir) + 513, read from the low bits of
// fma(dir, 512, 1.5 * 2^23), monotone in dir; the table is built with the same
// function. A codebook that is not strictly increasing, with a switch point
// outside (-1, 1), two switch points in one cell or one below 2^-60 in
// magnitude clears the table's flag, and its callers then use the scan.
//
// table_code() takes a direction from the same division the reference makes
// or, for a radius in the range where it is exact, from the Markstein
// quotient q0 + fma(-r, q0, y) / r with one correctly rounded reciprocal per
// vector (dir_markstein()).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace pqkv {

constexpr int kECells = 1024;           // direction cells over [-1, 1], 1/512 wide
constexpr int kECellSlots = kECells + 3;
constexpr int kECellOff = 513;          // cell of dir = round(512 dir) + 513
constexpr float kEMagic = 12582912.0f;  // 1.5 * 2^23: ulp 1, so fma(d, 512, kEMagic) holds round(512 d) in its low bits
constexpr float kEClamp = 1.001f;       // |dir| of the table path stays below; beyond, no switch point lies

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

// scan_index as a tree over register-held codebook values: the leftmost
// strict minimum of |d - c_i| over i < nl, then against the scan's start
// (1e30, index 0). The same index as the sequential scan for every d (the
// "keep the left one unless the right one is strictly smaller" rule is
// associative), with a 4-level instead of a 16-long dependency chain.
__device__ __forceinline__ int scan_index_tree(float d, const float (&c)[16], int nl) {
#pragma clang fp contract(off)
  float v[16];
  int ix[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    v[k] = k < nl ? fabsf(d - c[k]) : __builtin_inff();
    ix[k] = k;
  }
  auto level = [&](auto wc) {
    constexpr int W = decltype(wc)::value;
#pragma unroll
    for (int k = 0; k < 16; k += 2 * W) {
      const bool r = v[k + W] < v[k];
      v[k] = r ? v[k + W] : v[k];
      ix[k] = r ? ix[k + W] : ix[k];
    }
  };
  level(std::integral_constant<int, 1>{});
  level(std::integral_constant<int, 2>{});
  level(std::integral_constant<int, 4>{});
  level(std::integral_constant<int, 8>{});
  return v[0] < 1e30f ? ix[0] : 0;
}

// Direction cell, monotone in d: round(512 d) + 513, for |d| <= kEClamp in
// 0 .. kECellSlots - 1.
__device__ __forceinline__ uint32_t cell_bits(float d) {
  return __builtin_bit_cast(uint32_t, __builtin_fmaf(d, 512.0f, kEMagic));
}
__device__ __forceinline__ int dir_cell(float d) {
  return (int)(cell_bits(d) - __builtin_bit_cast(uint32_t, kEMagic)) + kECellOff;
}

// Order-preserving map between fp32 values and integers.
__device__ __forceinline__ int64_t fkey(float f) {
  const int32_t i = __builtin_bit_cast(int32_t, f);
  return i >= 0 ? (int64_t)i : -(int64_t)(i & 0x7FFFFFFF);
}
__device__ __forceinline__ float kfloat(int64_t k) {
  return k >= 0 ? __builtin_bit_cast(float, (int32_t)k) : __builtin_bit_cast(float, (int32_t)(0x80000000u | (uint32_t)(-k)));
}

// Workgroup barrier for LDS hand-offs: each wave waits for its own LDS
// operations only, so its global loads and global->LDS copies stay in flight
// across it (__syncthreads would drain them).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Builds the table for the nl-level codebook cb[0..15] (in LDS, written and
// made visible before the call) with a workgroup of NT >= 256 threads; all
// threads call it. On return (after a barrier) *table_ok says whether
// cells[] holds the table; thr[] and ucell[] are 16-entry LDS work arrays.
// Its barriers are LDS-only, so loads the caller issued before it keep
// running meanwhile.
template <int NT = 256>
__device__ __forceinline__ void build_cell_table(const float *cb, int nl, int tid, uint2 *cells, float *thr,
                                                 int *ucell, int *table_ok) {
  if (tid == 0) *table_ok = 1;
  lds_barrier();
  static_assert(NT >= 256 && NT % 64 == 0, "16 lanes for each of up to 15 switch points");
  // the codebook in registers for the scans
  float c[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) c[e] = cb[e];
  // Switch points: 16 lanes per point i, each the smallest fp32 d in
  // (c_i, c_{i+1}] that the scan maps to i + 1 or more. Once the scan maps
  // c_i to i or less and c_{i+1} to i + 1 or more (one lane each), that
  // holds for such d exactly when fl(c_{i+1} - d) < fl(d - c_i) (and below
  // the scan's 1e30 start): rounding is monotone, so every earlier centroid
  // is at least as far as c_i and every later one at least as far as
  // c_{i+1}. First, one probe: lane j tests the fp32 value j - 8 steps from
  // the midpoint of c_i and c_{i+1}, where the switch point lies up to the
  // subtractions' rounding for all but a pair around zero; when lane 0's
  // value fails and lane 15's passes, the first lane that passes holds it.
  // A pair symmetric about zero gets a second probe around half an ulp of
  // its centroids. Otherwise the lanes search 16-ary: lane j tests the (j + 1)/16 point of
  // the range, and the first that passes closes it (keys of fp32 values
  // differ by < 2^32, so 8 steps reach a range of one; a wave with no open
  // range leaves the loop).
  {
    const int i = tid >> 4, j = tid & 15;
    const bool act = i < nl - 1;
    const float ci = act ? cb[i] : 0.0f, cn = act ? cb[i + 1] : 0.0f;
    bool ok = false;
    {
      const bool bad = act && j < 2 && (j == 0 ? scan_index_tree(ci, c, nl) > i : scan_index_tree(cn, c, nl) < i + 1);
      ok = act && ci < cn && ((uint32_t)(__builtin_amdgcn_ballot_w64(bad) >> (16 * (i & 3))) & 3u) == 0;
    }
    auto pass = [&](int32_t key) {
#pragma clang fp contract(off)
      const float d = kfloat(key);
      const float en = cn - d, ei = d - ci;
      return en < ei && en < 1e30f;
    };
    // keys as unsigned differences (hi > lo, so hi - lo < 2^32 is exact
    // modulo 2^32) and lo + floor(span q / 16) without 64-bit products
    auto span_of = [](int32_t l, int32_t h) { return (uint32_t)h - (uint32_t)l; };
    auto part = [](uint32_t span, int q) { return (span >> 4) * (uint32_t)q + (((span & 15u) * (uint32_t)q) >> 4); };
    auto add = [](int32_t l, uint32_t off) { return (int32_t)((uint32_t)l + off); };
    int32_t lo = act ? (int32_t)fkey(ci) : 0, hi = act ? (int32_t)fkey(cn) : 0;
    const int32_t mid = act ? (int32_t)fkey(0.5f * ci + 0.5f * cn) : 0;
    // one probe of 16 consecutive keys from around - 8; closes the range
    // when the first key fails and the last passes
    auto probe = [&](int32_t around) {
      auto key_at = [&](int q) {
        const int64_t k = (int64_t)around - 8 + q;
        return (int32_t)(k < lo ? lo : k > hi ? hi : k);
      };
      const bool open = ok && span_of(lo, hi) > 1u;
      const bool pp = open && pass(key_at(j));
      const uint32_t pm = (uint32_t)(__builtin_amdgcn_ballot_w64(pp) >> (16 * (i & 3))) & 0xFFFFu;
      if (open && (pm & 1u) == 0 && (pm >> 15) != 0) {
        hi = key_at(__builtin_ctz(pm));
        lo = add(hi, 0xFFFFFFFFu);   // hi - 1
      }
    };
    probe(mid);
    // A pair symmetric about zero (c_i = -c_{i+1}, midpoint 0): the switch
    // point is where fl(c_{i+1} - d) or fl(-c_i + d) first rounds away from
    // its centroid, half an ulp of it (the smaller of the ulp below c_{i+1}
    // and the ulp above -c_i), up to the tie rule.
    if (__builtin_amdgcn_ballot_w64(ok && span_of(lo, hi) > 1u) != 0) {
      const float ub = cn - kfloat((int64_t)fkey(cn) - 1), ua = kfloat((int64_t)fkey(-ci) + 1) + ci;
      probe(act && mid == 0 ? (int32_t)fkey(0.5f * (ub < ua ? ub : ua)) : mid);
    }
    for (int step = 0; step < 10; ++step) {
      const bool open = ok && span_of(lo, hi) > 1u;
      if (__builtin_amdgcn_ballot_w64(open) == 0) break;
      const uint32_t span = span_of(lo, hi);
      const int32_t cand = j == 15 ? hi : add(lo, part(span, j + 1));
      const bool p = open && pass(cand);
      const uint32_t gm = (uint32_t)(__builtin_amdgcn_ballot_w64(p) >> (16 * (i & 3))) & 0xFFFFu;
      const int k = gm ? __builtin_ctz(gm) : 15;
      if (open) {
        const int32_t nhi = k == 15 ? hi : add(lo, part(span, k + 1));
        lo = k == 0 ? lo : add(lo, part(span, k));
        hi = nhi;
      }
    }
    if (act && j == 0) {
      if (!ok || span_of(lo, hi) != 1u) {
        *table_ok = 0;
      } else {
        const float t = kfloat(hi);
        thr[i] = t;
        if (!(fabsf(t) >= 0x1p-60f) || !(fabsf(t) < 1.0f)) *table_ok = 0;
        else ucell[i] = dir_cell(t);
      }
    }
  }
  lds_barrier();
  if (*table_ok != 0) {
    // the switch points' cells in registers (read once: the table stores
    // below could alias them); cells past the last switch point match no slot
    int uc[15];
#pragma unroll
    for (int e = 0; e < 15; ++e) uc[e] = e < nl - 1 ? ucell[e] : 0x7FFFFFFF;
    // index at each cell's start: the switch points in earlier cells
    // (branch-free); the switch point inside a cell is written below
    for (int u = tid; u < kECellSlots; u += NT) {
      int base = 0;
#pragma unroll
      for (int e = 0; e < 15; ++e) base += uc[e] < u ? 1 : 0;
      cells[u] = make_uint2((uint32_t)base, 0x7F800000u);   // +inf: no switch point inside
    }
    // two switch points in one cell: no table (the cells are non-decreasing)
    bool crowded = false;
#pragma unroll
    for (int e = 0; e + 1 < 15; ++e) crowded |= e + 1 < nl - 1 && uc[e] == uc[e + 1];
    lds_barrier();
    if (crowded) {
      if (tid == 0) *table_ok = 0;
    } else if (tid < nl - 1) {
      cells[ucell[tid]].y = __builtin_bit_cast(uint32_t, thr[tid]);
    }
  }
  lds_barrier();
}

// Radii for which the Markstein quotient gives the reference's index:
// zero-like (dir = 0, reached through inv = 0 on finite y) or finite and
// >= 2^-40 (quotient exact wherever a switch point is within a factor of two,
// |dir| <= 1 + 11 ulp).
__device__ __forceinline__ bool markstein_radius(float r) {
  return r <= 1e-30f || (r >= 0x1p-40f && r < __builtin_inff());
}

// dir = RN(y / r) for a radius markstein_radius() accepts, inv = RN(1 / r)
// (0 for a zero-like radius).
__device__ __forceinline__ float dir_markstein(float y, float r, float inv) {
#pragma clang fp contract(off)
  const float q0 = y * inv;
  const float e = __builtin_fmaf(-r, q0, y);
  return __builtin_fmaf(e, inv, q0);
}

// dir = RN(y / r) by division, mapped into the table's range: NaN to -2
// (index 0, as the scan gives), then clamped to +-kEClamp.
__device__ __forceinline__ float dir_divided(float y, float r) {
  float d = r > 1e-30f ? __fdiv_rn(y, r) : 0.0f;
  d = d == d ? d : -2.0f;
  return __builtin_fminf(__builtin_fmaxf(d, -kEClamp), kEClamp);
}

__device__ __forceinline__ int table_code(const uint2 *cells, float d) {
  const uint2 ce = cells[dir_cell(d)];
  return (int)ce.x + (d >= __builtin_bit_cast(float, ce.y) ? 1 : 0);
}

}  // namespace pqkv
