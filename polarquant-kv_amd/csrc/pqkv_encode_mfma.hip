// Fast fused encoder on the matrix cores (gfx950) for fp16 input vectors:
// rotate, radius, direction, nearest centroid, block_pq4 / block_pq2 packing.
//
// Work split. A workgroup of four waves takes 64 vectors per step. The
// step's input (64 x d fp16) arrives in LDS by direct global->LDS copies
// issued one step ahead, and every wave reads all of it as the B operand of
// v_mfma_f32_16x16x32_f16 (B = X^T, 16 vectors per tile). Wave w computes a
// quarter of the output coordinates, j = 16 k + 4 w + i (i = 0..3,
// k = 0..d/16-1), so its A operand (those d/4 rows of R, split as
// R = R_hi + R_lo in fp16, the fp16 input being exact) stays in registers for
// the whole launch: two MFMAs per tile product give fp32-grade rotated values
// (not the FMA-chain rounding of the exact encoder; the quantiser below is
// bit-exact on the values this rotation produces).
//
// Radius: the reference's tree of squares (slot t += slot t + s for
// s = 64 .. 1, csrc/flash_turboquant.cu:141-147) with the coordinate split
// above: the steps s >= 16 pair coordinates of one wave (k bit 2 in-lane,
// k bits 1 and 0 across the permlane32 / permlane16 swaps; IEEE addition
// commutes, so both lanes of a swap hold the same sum), which leaves wave w
// with slots 4 w + i. Those 16 partial sums per vector go through LDS, and
// lane L of every wave finishes the steps s = 8 .. 1 of vector L.
//
// Nearest centroid: the switch-point cell table of pqkv_cells.h, built by
// each workgroup at launch (the scan when the codebook does not allow it).
// The direction is the Markstein quotient (one correctly rounded 1 / r per
// vector): RN(y / r) whenever its residual is exact, which holds when
// exp(r) + exp(q0) - 46 >= -149. That form is taken per 64-vector step
// when every radius is finite and >= 2^-40 (or zero-like, dir = 0): then
// every direction within a factor of two of a switch point (>= 2^-60) is
// exact, and a direction off by an ulp elsewhere crosses no switch point, so
// the index is the reference's. Steps with other radii divide per coordinate.
//
// Output: each wave writes its codes (and wave w the radius of block w) into
// an LDS copy of the step's blocks, stored to memory one step later with
// 16-byte writes (dword writes for strided rows).
//
// QJL keys (m = d projections): the quantiser also writes the residual
// e = y - r c[code] (fp32 r) times 1 / r into LDS as fp16 hi / lo planes, and
// one step later wave w computes projections (d / 4) w .. of P_rot e on the
// matrix cores (P_rot = P R^T split hi / lo in registers like R; three
// products per tile product, ~2^-21 relative) and packs sign bit m =
// (P_rot e)[m] >= 0, LSB first. Scaling e by 1 / r keeps the fp16 planes in
// range and leaves every sign as it is. Steps are 32 vectors there (register
// and LDS room for P).
//
// Schedule: a software pipeline with one workgroup barrier per step. While
// a wave's matrix-core products rotate step k, its vector ALUs quantise step
// k - 1 (rotation held in registers); step k + 1's input is in flight and
// step k - 2's blocks are being written.
#include "pqkv_cells.h"
#include "pqkv_device.h"
#include "pqkv_launch.h"

namespace pqkv {

namespace {

#ifndef PQKV_ENC_TILES
#define PQKV_ENC_TILES 4
#endif
#ifndef PQKV_ENC_VALU_PER_MFMA
#define PQKV_ENC_VALU_PER_MFMA 2
#endif
#ifndef PQKV_ENC_BLOCKS
#define PQKV_ENC_BLOCKS 2
#endif
constexpr int kEW = 4;              // waves per workgroup
constexpr int kET = PQKV_ENC_TILES; // 16-vector tiles per workgroup step
constexpr int kEG = 16 * kET;       // vectors per workgroup step
constexpr int kEBlocksPerCU = PQKV_ENC_BLOCKS;  // resident workgroups per compute unit
constexpr int kEPart = 20;          // floats per vector in the partial-sum exchange (16 used; 80-byte rows
                                    // put the 16-byte reads of lanes 0..15 in distinct banks)

__device__ __forceinline__ float4_t mfma16(half8_t a, half8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}


// Two tree steps at once: after v_permlane32_swap of a and b, lane L < 32
// holds a[L] + a[L + 32] and lane L >= 32 holds b[L - 32] + b[L].
__device__ __forceinline__ float swap32_pair_add(float a, float b) {
  auto s = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b), false, false);
  return __builtin_bit_cast(float, (uint32_t)s[0]) + __builtin_bit_cast(float, (uint32_t)s[1]);
}
// After v_permlane16_swap of a and b (rows of 16 lanes): row 0 holds
// a[r0] + a[r1], row 1 b[r0] + b[r1], row 2 a[r2] + a[r3], row 3 b[r2] + b[r3].
__device__ __forceinline__ float swap16_pair_add(float a, float b) {
  auto s = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b), false, false);
  return __builtin_bit_cast(float, (uint32_t)s[0]) + __builtin_bit_cast(float, (uint32_t)s[1]);
}

__device__ __forceinline__ float bperm_f(int src_lane, float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src_lane * 4, __builtin_bit_cast(int, v)));
}

template <bool B>
struct TableFlag {
  static constexpr bool on = B;
};

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) uint8_t lds_u8;

// LDS stores issued while the next step's copies into xs are in flight (the
// stage copy of a step's blocks, the radius partial sums). Written as
// instructions the compiler's wait tracking does not see: it would otherwise
// wait for those copies (which never overlap these buffers) and for the
// block stores before each LDS store. The workgroup barrier that follows the
// stores waits for them (lgkmcnt 0); as volatile asm they stay in order with
// it.
__device__ __forceinline__ void lds_st32(__attribute__((address_space(3))) float *p, float v) {
  asm volatile("ds_write_b32 %0, %1" ::"v"((uint32_t)(uintptr_t)p), "v"(v));
}
__device__ __forceinline__ void lds_st64(__attribute__((address_space(3))) half_t *p, uint64_t v) {
  asm volatile("ds_write_b64 %0, %1" ::"v"((uint32_t)(uintptr_t)p), "v"(v));
}
__device__ __forceinline__ uint32_t pack_h2(half_t a, half_t b) {
  half2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ void stage_st16(lds_u8 *p, uint32_t v) {
  asm volatile("ds_write_b16 %0, %1" ::"v"((uint32_t)(uintptr_t)p), "v"(v));
}
__device__ __forceinline__ void stage_st8(lds_u8 *p, uint32_t v) {
  asm volatile("ds_write_b8 %0, %1" ::"v"((uint32_t)(uintptr_t)p), "v"(v));
}
typedef __attribute__((address_space(3))) half8_t lds_half8;
typedef __attribute__((address_space(3))) float4_t lds_float4;

}  // namespace

template <int D, int BITS, bool QJL>
__global__ void __launch_bounds__(kEW * 64, kEBlocksPerCU) encode_mfma_kernel(const EncodeArgs a, float *rot_out,
                                                                                float *radius_out) {
  constexpr int ET = QJL ? 2 : kET;      // 16-vector tiles per step (QJL: register and LDS room for P)
  constexpr int EG = 16 * ET;            // vectors per step
  constexpr int KS = D / 32;             // k-steps over input coordinates
  constexpr int MTW = D / 64;            // 16-row output tiles per wave
  constexpr int NL = 1 << BITS;
  constexpr int BB = block_bytes(BITS);
  constexpr int VB = vector_bytes(D, BITS);
  constexpr int XB = 2 * D;              // input bytes per vector
  constexpr int CH = XB / 16;            // 16-byte chunks per vector
  constexpr int VPI = 1024 / XB;         // vectors per wave copy instruction (64 lanes x 16 bytes)
  constexpr int NCOPY = EG / VPI;       // copy instructions per step
  constexpr int DW = VB / 4;             // output dwords per vector
  constexpr int SB = D / 8;              // sign bytes per vector (m = d projections)
  __shared__ __attribute__((aligned(16))) uint8_t xs[2][EG * XB];
  __shared__ __attribute__((aligned(16))) float part[2][EG * kEPart];
  __shared__ __attribute__((aligned(16))) uint8_t stage[2][EG * VB];
  // QJL: the step's rotated residuals scaled by 1 / r, as the B operand of the
  // sign product (fp16 hi / lo planes, chunk-swizzled like xs), and the
  // step's sign bytes
  __shared__ __attribute__((aligned(16))) half_t ebuf[2][QJL ? 2 * EG * D : 8];
  __shared__ __attribute__((aligned(16))) uint8_t sstage[2][QJL ? EG * SB : 16];
  __shared__ uint2 cells[kECellSlots];   // (index at the cell start, switch point bits or +inf)
  __shared__ float cb[16], thr[16];
  __shared__ int ucell[16];
  __shared__ int table_ok;
  typedef __attribute__((address_space(3))) uint32_t lds_u32;

  const int tid = threadIdx.x, lane = tid & 63;
  // the codebook's load first: its LDS copy below then waits for it alone,
  // not for R's loads behind it
  const float cbv = tid < NL ? a.codebook[tid] : 0.0f;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;
  // chunk swizzle of a vector's 16-byte pieces in LDS: the B-operand reads of
  // lanes 0..15 (16 vectors, one chunk each) land in distinct banks
  auto swz = [](int vl) { return D == 128 ? (vl & 15) : ((vl >> 1) & 7); };

  // ---- A operand, in registers for the launch: row p of tile mt is output
  // coordinate j = 16 (4 mt + p / 4) + 4 wave + p % 4; lane (p, grp) holds
  // R[j][32 ks + 8 grp .. + 7] ----
  // (loaded here, split after the set-up below so that the loads' latency
  // overlaps it)
  half8_t ah[MTW][KS], al[MTW][KS];
  float4_t rraw[MTW][KS][2];
#pragma unroll
  for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int j = 16 * (4 * mt + (col >> 2)) + 4 * wave + (col & 3);
      const float4_t *rr = (const float4_t *)(a.R + (int64_t)j * D + 32 * ks + 8 * grp);
      rraw[mt][ks][0] = rr[0];
      rraw[mt][ks][1] = rr[1];
    }
  auto split_r = [&] {
#pragma unroll
    for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float rv = rraw[mt][ks][e >> 2][e & 3];
          const half_t h = (half_t)rv;
          ah[mt][ks][e] = h;
          al[mt][ks][e] = (half_t)(rv - (float)h);
        }
  };
  // QJL: P_rot = P R^T as the A operand of the sign product, the same way:
  // row p of tile mt is projection (d / 4) wave + 16 mt + p
  half8_t ph[QJL ? MTW : 1][KS], pl[QJL ? MTW : 1][KS];
  if constexpr (QJL) {
#pragma unroll
    for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int mrow = (D / 4) * wave + 16 * mt + col;
        const float4 *pr = (const float4 *)(a.p_rot + (int64_t)mrow * D + 32 * ks + 8 * grp);
        const float4 r0 = pr[0], r1 = pr[1];
        const float rv[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const half_t h = (half_t)rv[e];
          ph[mt][ks][e] = h;
          pl[mt][ks][e] = (half_t)(rv[e] - (float)h);
        }
      }
  }

  if (tid < 16) cb[tid] = cbv;

  const half_t *x = (const half_t *)a.x;
  // vector v = n_inner * vo + vi; the host keeps n below 2^32 (a single row
  // has n_inner = n, so vo = 0 there)
  const uint32_t n = (uint32_t)(a.n_outer * a.n_inner);
  const int64_t groups = ((int64_t)n + EG - 1) / EG;
  const FastDiv by_inner((uint32_t)a.n_inner);
  auto split = [&](uint32_t v, uint32_t &vo, uint32_t &vi) {
    vo = by_inner.div(v);
    vi = v - vo * (uint32_t)a.n_inner;
  };
  // Step g's input into xs[b]: copy instruction q covers vectors q VPI ..,
  // lane L piece L % CH of vector q VPI + L / CH, which holds chunk
  // (L % CH) ^ swz(vector). Lanes past the end copy the last vector again
  // (into slots no step reads), so the copies need no branch.
  static_assert(NCOPY % kEW == 0, "copy instructions split evenly over the waves");
  // One contiguous run of vectors (n_outer <= 1): a whole step's copy
  // sources are the step's base (uniform) plus per-lane byte offsets that
  // do not change from step to step.
  // (not for the QJL kernels, which have no registers to spare for it)
  const bool run_x = !QJL && a.n_outer <= 1;
  uint32_t xoff[NCOPY / kEW];
#pragma unroll
  for (int j = 0; j < NCOPY / kEW; ++j) {
    const int vl = (wave + kEW * j) * VPI + lane / CH;
    xoff[j] = (uint32_t)(vl * XB + 16 * ((lane % CH) ^ swz(vl)));
  }
  auto issue = [&](int64_t g, int b) {
    if (!QJL && run_x && (uint32_t)g * EG + EG <= n) {
      const uint8_t *base = (const uint8_t *)x + (int64_t)g * EG * XB;
#pragma unroll
      for (int j = 0; j < NCOPY / kEW; ++j)
        __builtin_amdgcn_global_load_lds((const void *)(base + xoff[j]), (lds_void *)(xs[b] + 1024 * (wave + kEW * j)),
                                         16, 0, 0);
      return;
    }
#pragma unroll
    for (int j = 0; j < NCOPY / kEW; ++j) {
      const int q = wave + kEW * j;
      const int vl = q * VPI + lane / CH;
      uint32_t vo, vi;
      split(min((uint32_t)g * EG + vl, n - 1), vo, vi);
      const half_t *row = x + (int64_t)vo * a.x_outer_stride + (int64_t)vi * D;
      __builtin_amdgcn_global_load_lds((const void *)(row + 8 * ((lane % CH) ^ swz(vl))), (lds_void *)(xs[b] + 1024 * q),
                                       16, 0, 0);
    }
  };
  // Step g's blocks from stage[sb] to memory: one run of 16-byte pieces when
  // the blocks are one aligned run, else dword by dword.
  const bool run16 = a.n_outer <= 1 && a.pages == nullptr && ((uintptr_t)a.blocks & 15) == 0;
  auto flush = [&](int64_t g, int sb) {
    const lds_u8 *stg = (const lds_u8 *)stage[sb];
    if (run16) {
      const uint32_t v0 = (uint32_t)g * EG;
      const int nbytes = (int)min(n - v0, (uint32_t)EG) * VB;
      uint8_t *base = a.blocks + (int64_t)v0 * VB;
#pragma unroll
      for (int it = 0; it < (EG * VB / 16 + kEW * 64 - 1) / (kEW * 64); ++it) {
        const int p = tid + kEW * 64 * it;
        if (16 * p + 16 <= nbytes) {
          *(u32x4 *)(base + 16 * p) = *(const __attribute__((address_space(3))) u32x4 *)(stg + 16 * p);
        } else if (16 * p < nbytes) {
          for (int c = 0; c < 4 && 16 * p + 4 * c < nbytes; ++c)
            *(uint32_t *)(base + 16 * p + 4 * c) = *(const lds_u32 *)(stg + 16 * p + 4 * c);
        }
      }
      return;
    }
#pragma unroll
    for (int it = 0; it < (EG * DW + kEW * 64 - 1) / (kEW * 64); ++it) {
      const int q = tid + kEW * 64 * it;
      if (q < EG * DW) {
        const int vl = q / DW, c = q - vl * DW;
        const uint32_t v = (uint32_t)g * EG + vl;
        if (v < n) {
          uint32_t vo, vi;
          split(v, vo, vi);
          const uint32_t w = *(const lds_u32 *)(stg + vl * VB + 4 * c);
          *(uint32_t *)(encode_out_addr(a, a.blocks, a.pages, a.blocks_outer_stride, vo, vi, VB) + 4 * c) = w;
        }
      }
    }
  };
  // Workgroup barrier for LDS hand-offs: unlike __syncthreads it does not
  // wait for this wave's copies and stores still in flight.
  auto barrier = [] { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };
  // Wait for this wave's copies and stores (the builtin, which the
  // compiler's wait tracking sees: vmcnt 0).
  auto wait_mem = [] { __builtin_amdgcn_s_waitcnt(0x0F70); };

  typedef float4_t Tile[ET][MTW];
  // ---- rotation of the step in xs[b]: y[t][mt] = rows of tile mt for
  // vectors 16 t + col ----
  auto rotate = [&](int b, Tile &y) {
#pragma unroll
    for (int t = 0; t < ET; ++t)
#pragma unroll
      for (int mt = 0; mt < MTW; ++mt) y[t][mt] = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < ET; ++t)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int vl = 16 * t + col;
        const half8_t xb = *(const lds_half8 *)(xs[b] + vl * XB + 16 * ((4 * ks + grp) ^ swz(vl)));
#pragma unroll
        for (int mt = 0; mt < MTW; ++mt) {
          y[t][mt] = mfma16(ah[mt][ks], xb, y[t][mt]);
          y[t][mt] = mfma16(al[mt][ks], xb, y[t][mt]);
        }
      }
  };
  // ---- radius tree, steps s >= 16 in the wave, into part[pb]: slots
  // 4 wave + i. The swaps pair lanes grp, grp ^ 2 (s = 32) and grp, grp ^ 1
  // (s = 16) for two slots at a time, leaving slot i = 2 (grp & 1) + grp / 2
  // in lane (col, grp). ----
  const int my_slot = 2 * (grp & 1) + (grp >> 1);
  auto tree = [&](const Tile &y, int pb) {
#pragma unroll
    for (int t = 0; t < ET; ++t) {
      float z;
      {
#pragma clang fp contract(off)
        float s[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          s[i] = y[t][0][i] * y[t][0][i];
          if constexpr (MTW == 2) s[i] = s[i] + y[t][1][i] * y[t][1][i];  // s = 64
        }
        const float s01 = swap32_pair_add(s[0], s[1]);  // s = 32: slot 0 (lanes < 32), slot 1
        const float s23 = swap32_pair_add(s[2], s[3]);  // slot 2, slot 3
        z = swap16_pair_add(s01, s23);                  // s = 16
      }
      lds_st32((__attribute__((address_space(3))) float *)part[pb] + (16 * t + col) * kEPart + 4 * wave + my_slot, z);
    }
  };
  // ---- lane L: steps s = 8 .. 1 of vector L (lanes L mod EG) of step g
  // from part[pb], its radius (into stage[sb]) and 1 / r; whether the whole
  // step takes the table's fast form ----
  auto finish = [&](int64_t g, int pb, int sb, float &r, float &inv) -> bool {
    const int lv = lane % EG;
    const uint32_t vme = (uint32_t)g * EG + lv;
    bool fast;
    {
#pragma clang fp contract(off)
      const float *pp = part[pb] + lv * kEPart;
      const float4_t p0 = *(const lds_float4 *)(pp), p1 = *(const lds_float4 *)(pp + 4);
      const float4_t p2 = *(const lds_float4 *)(pp + 8), p3 = *(const lds_float4 *)(pp + 12);
      // slots 0..15 = p0 p1 p2 p3; s = 8: t += t + 8
      const float q0 = p0[0] + p2[0], q1 = p0[1] + p2[1], q2 = p0[2] + p2[2], q3 = p0[3] + p2[3];
      const float q4 = p1[0] + p3[0], q5 = p1[1] + p3[1], q6 = p1[2] + p3[2], q7 = p1[3] + p3[3];
      const float u0 = q0 + q4, u1 = q1 + q5, u2 = q2 + q6, u3 = q3 + q7;  // s = 4
      const float w0 = u0 + u2, w1 = u1 + u3;                             // s = 2
      const float tot = w0 + w1;                                          // s = 1
      r = (float)__builtin_sqrt((double)tot);
      const bool nz = r > 1e-30f;
      inv = nz ? __fdiv_rn(1.0f, r) : 0.0f;
      // zero-like (dir = 0, reached through inv = 0 on finite y) or finite
      // and >= 2^-40 (Markstein quotient exact, |dir| <= 1 + 11 ulp)
      fast = markstein_radius(r);
    }
    if (vme < n && lane < EG) {
      if (wave < D / 32) stage_st16((lds_u8 *)stage[sb] + lv * VB + wave * BB, radius_half_bits(r));
      if (radius_out != nullptr && wave == 0) radius_out[vme] = r;
    }
    return __builtin_amdgcn_ballot_w64(!fast && vme < n) == 0;
  };
  // ---- directions, indices, packing of step g (rotation y, radii r / inv
  // held by lane 16 t + col) into stage[sb] ----
  auto quantise = [&](auto table_flag, auto fast_flag, const Tile &y, int sb, float r, float inv) {
    constexpr bool kTable = decltype(table_flag)::on;
    constexpr bool kFast = decltype(fast_flag)::on;
#pragma unroll
    for (int t = 0; t < ET; ++t) {
      const int vl = 16 * t + col;
      const float rt = bperm_f(vl, r), it = bperm_f(vl, inv);
      const bool nzt = rt > 1e-30f;
      int code[MTW][4];
      auto dir_of = [&](float yv) {
        if constexpr (kFast) return dir_markstein(yv, rt, it);
        else return dir_divided(yv, rt);
      };
      if constexpr (kTable && QJL) {
        // (one coordinate at a time: the QJL kernels have no registers to
        // spare for the batched form below)
#pragma unroll
        for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            code[mt][i] = table_code(cells, dir_of(y[t][mt][i]));
          }
      } else if constexpr (kTable) {
        // in three passes over the tile's coordinates (directions, cell
        // reads, codes), so that the lane's cell reads are in flight
        // together instead of each waiting for the one before
        float dv[MTW][4];
#pragma unroll
        for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i) dv[mt][i] = dir_of(y[t][mt][i]);
        uint2 ce[MTW][4];
#pragma unroll
        for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i) ce[mt][i] = cells[dir_cell(dv[mt][i])];
#pragma unroll
        for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            code[mt][i] = (int)ce[mt][i].x + (dv[mt][i] >= __builtin_bit_cast(float, ce[mt][i].y) ? 1 : 0);
      } else {
#pragma unroll
        for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float d = nzt ? __fdiv_rn(y[t][mt][i], rt) : 0.0f;
            code[mt][i] = scan_index_rolled(d, cb, NL);
          }
      }
      if constexpr (QJL) {
        // residual e = y - r c[code] (fp32 r), times 1 / r (the signs do not
        // change; fp16 planes cannot hold e itself), into ebuf[sb]: four
        // coordinates 16 (4 mt + grp) + 4 wave .. + 3 per (lane, mt)
#pragma unroll
        for (int mt = 0; mt < MTW; ++mt) {
          half_t hv[4], lv[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float e = __builtin_fmaf(-rt, cb[code[mt][i]], y[t][mt][i]) * it;
            hv[i] = (half_t)e;
            lv[i] = (half_t)(e - (float)hv[i]);
          }
          const int j0 = 16 * (4 * mt + grp) + 4 * wave;
          const int off = vl * D + 8 * ((j0 >> 3) ^ swz(vl)) + (j0 & 7);
          const uint64_t hq = (uint64_t)pack_h2(hv[0], hv[1]) | ((uint64_t)pack_h2(hv[2], hv[3]) << 32);
          const uint64_t lq = (uint64_t)pack_h2(lv[0], lv[1]) | ((uint64_t)pack_h2(lv[2], lv[3]) << 32);
          lds_st64((__attribute__((address_space(3))) half_t *)ebuf[sb] + off, hq);
          lds_st64((__attribute__((address_space(3))) half_t *)ebuf[sb] + EG * D + off, lq);
        }
      }
      // coordinate j = 16 k + 4 wave + i, k = 4 mt + grp: block k / 2,
      // qs byte 8 (k & 1) + 2 wave + i / 2 (4-bit) or 4 (k & 1) + wave (2-bit)
#pragma unroll
      for (int mt = 0; mt < MTW; ++mt) {
        lds_u8 *dst = (lds_u8 *)stage[sb] + vl * VB + (2 * mt + (grp >> 1)) * BB + 2;
        if constexpr (BITS == 4) {
          const uint32_t h = (uint32_t)(code[mt][0] | (code[mt][1] << 4) | (code[mt][2] << 8) | (code[mt][3] << 12));
          stage_st16(dst + 8 * (grp & 1) + 2 * wave, h);
        } else {
          const uint32_t h = (uint32_t)(code[mt][0] | (code[mt][1] << 2) | (code[mt][2] << 4) | (code[mt][3] << 6));
          stage_st8(dst + 4 * (grp & 1) + wave, h);
        }
      }
    }
  };
  auto store_rot = [&](const Tile &y, int64_t g) {
    if (rot_out == nullptr) return;
#pragma unroll
    for (int t = 0; t < ET; ++t) {
      const uint32_t vg = (uint32_t)g * EG + 16 * t + col;
      if (vg < n) {
#pragma unroll
        for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i) rot_out[(int64_t)vg * D + 16 * (4 * mt + grp) + 4 * wave + i] = y[t][mt][i];
      }
    }
  };

  const int64_t g_step = gridDim.x;  // a workgroup's steps are blockIdx.x + k gridDim.x

  // ---- QJL sign product of the step whose residuals are in ebuf[eb]: wave
  // w takes projections (d / 4) w .. + d / 4 - 1 (three products per tile,
  // P_hi e_hi + P_hi e_lo + P_lo e_hi); bit m of a vector's signs is
  // (P_rot e)[m] >= 0, LSB first, into sstage[sb] ----
  auto sign_product = [&](int eb, int sb) {
#pragma unroll
    for (int t = 0; t < ET; ++t) {
      const int vl = 16 * t + col;
      float4_t sacc[MTW];
#pragma unroll
      for (int mt = 0; mt < MTW; ++mt) sacc[mt] = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int off = vl * D + 8 * ((4 * ks + grp) ^ swz(vl));
        const half8_t eh = *(const lds_half8 *)(ebuf[eb] + off);
        const half8_t el = *(const lds_half8 *)(ebuf[eb] + EG * D + off);
#pragma unroll
        for (int mt = 0; mt < MTW; ++mt) {
          sacc[mt] = mfma16(ph[mt][ks], eh, sacc[mt]);
          sacc[mt] = mfma16(ph[mt][ks], el, sacc[mt]);
          sacc[mt] = mfma16(pl[mt][ks], eh, sacc[mt]);
        }
      }
      // lane (col, grp) holds projections (d / 4) w + 16 mt + 4 grp + i:
      // bits 4 (grp & 1) + i of sign byte (d / 32) w + 2 mt + grp / 2
#pragma unroll
      for (int mt = 0; mt < MTW; ++mt) {
        const uint32_t nib = (sacc[mt][0] >= 0.0f ? 1u : 0u) | (sacc[mt][1] >= 0.0f ? 2u : 0u) |
                             (sacc[mt][2] >= 0.0f ? 4u : 0u) | (sacc[mt][3] >= 0.0f ? 8u : 0u);
        const uint32_t other = (uint32_t)__shfl_xor((int)nib, 16, 64);
        if ((grp & 1) == 0)
          stage_st8((lds_u8 *)sstage[sb] + vl * SB + (D / 32) * wave + 2 * mt + (grp >> 1), nib | (other << 4));
      }
    }
  };
  const bool run16q = a.n_outer <= 1 && a.pages == nullptr && ((uintptr_t)a.qjl & 15) == 0;
  auto flush_signs = [&](int64_t g, int sb) {
    const lds_u8 *stg = (const lds_u8 *)sstage[sb];
    if (run16q) {
      const uint32_t v0 = (uint32_t)g * EG;
      const int nbytes = (int)min(n - v0, (uint32_t)EG) * SB;
      uint8_t *base = a.qjl + (int64_t)v0 * SB;
      const int p = tid;
      if (16 * p + 16 <= nbytes) {
        *(u32x4 *)(base + 16 * p) = *(const __attribute__((address_space(3))) u32x4 *)(stg + 16 * p);
      } else if (16 * p < nbytes) {
        for (int c = 0; c < 4 && 16 * p + 4 * c < nbytes; ++c)
          *(uint32_t *)(base + 16 * p + 4 * c) = *(const lds_u32 *)(stg + 16 * p + 4 * c);
      }
      return;
    }
    const int q = tid;  // dword q of the step's signs
    if (q < EG * SB / 4) {
      const int vl = q / (SB / 4), c = q - vl * (SB / 4);
      const uint32_t v = (uint32_t)g * EG + vl;
      if (v < n) {
        uint32_t vo, vi;
        split(v, vo, vi);
        *(uint32_t *)(encode_out_addr(a, a.qjl, a.qjl_pages, a.qjl_outer_stride, vo, vi, SB) + 4 * c) =
            *(const lds_u32 *)(stg + vl * SB + 4 * c);
      }
    }
  };
  static_assert(!QJL || EG * SB <= 16 * kEW * 64, "one 16-byte piece of signs per thread");

  // QJL keys: the same pipeline one stage deeper. Iteration k rotates step
  // g_k, quantises g_{k-1} (codes, and its residuals into ebuf[k & 1]), runs
  // the sign product of g_{k-2} from ebuf[(k - 1) & 1] into sstage[k & 1],
  // stores the blocks of g_{k-2} and the signs of g_{k-3}.
  auto run_qjl = [&](auto table_flag) {
    constexpr bool kTable = decltype(table_flag)::on;
    const int64_t g0 = blockIdx.x;
    const int64_t steps = (groups - g0 + g_step - 1) / g_step;  // this workgroup's steps
    Tile acc, accp;   // (step g0's input was issued before the set-up)
    for (int64_t k = 0; k < steps + 3; ++k) {
      const int b = (int)(k & 1);
      const int64_t gk = g0 + k * g_step;
#pragma unroll
      for (int t = 0; t < ET; ++t)
#pragma unroll
        for (int mt = 0; mt < MTW; ++mt) accp[t][mt] = acc[t][mt];
      wait_mem();
      barrier();
      if (k >= 2 && k - 2 < steps) flush(gk - 2 * g_step, b ^ 1);
      if (k >= 3 && k - 3 < steps) flush_signs(gk - 3 * g_step, b ^ 1);
      float r = 0.f, inv = 0.f;
      bool step_fast = true;
      if (k >= 1 && k - 1 < steps) step_fast = finish(gk - g_step, b ^ 1, b, r, inv);
      if (k >= 2 && k - 2 < steps) sign_product(b ^ 1, b);
      if (k < steps) {
        rotate(b, acc);
        issue(k + 1 < steps ? gk + g_step : gk, b ^ 1);
      }
      if (k >= 1 && k - 1 < steps) {
        if (!kTable || step_fast) quantise(table_flag, TableFlag<true>{}, accp, b, r, inv);
        else quantise(table_flag, TableFlag<false>{}, accp, b, r, inv);
      }
      if (k < steps) tree(acc, b);
    }
  };

  // Software pipeline over the workgroup's steps g0, g0 + G, ...: iteration k
  // rotates step g_k (input in xs[k & 1], tree partials into part[k & 1]),
  // copies step g_{k+1} into xs[(k + 1) & 1], quantises step g_{k-1} (rotation
  // kept in registers, partials from part[(k - 1) & 1]) into stage[k & 1] and
  // stores step g_{k-2} from stage[(k - 2) & 1]: one workgroup barrier per
  // step, and each wave's matrix-core products of one step run beside its
  // quantiser arithmetic of the step before.
  auto run = [&](auto table_flag) {
    constexpr bool kTable = decltype(table_flag)::on;
    int64_t g = blockIdx.x;
    Tile acc, accp;   // (step g's input was issued before the set-up)
    wait_mem();
    barrier();
    rotate(0, acc);
    if (g + g_step < groups) issue(g + g_step, 1);
    tree(acc, 0);
    store_rot(acc, g);
    int64_t gp = g, gpp = -1;
    int k = 1;
    for (g += g_step; g < groups; g += g_step, ++k) {
      const int b = k & 1;
#pragma unroll
      for (int t = 0; t < ET; ++t)
#pragma unroll
        for (int mt = 0; mt < MTW; ++mt) accp[t][mt] = acc[t][mt];
      wait_mem();
      barrier();  // xs[b], part[b ^ 1] and stage[b ^ 1] complete; xs[b ^ 1], part[b], stage[b] free
      if (gpp >= 0) flush(gpp, b ^ 1);
      float r, inv;
      const bool step_fast = finish(gp, b ^ 1, b, r, inv);
      // the step whose input goes into xs[b ^ 1]: the next one, or this one
      // again at the end (a copy nothing reads), so the body has no branch
      const int64_t g_next = g + g_step < groups ? g + g_step : g;
      auto body = [&](auto fast_flag) {
        rotate(b, acc);
        // the next step's copies go out after this step's reads of xs:
        // issued earlier, the compiler would wait for them before the reads
        // (it cannot tell xs[b] from xs[b ^ 1])
        issue(g_next, b ^ 1);
        quantise(table_flag, fast_flag, accp, b, r, inv);
        tree(acc, b);
        // interleave the rotation's matrix-core products with the previous
        // step's quantiser arithmetic: one product, then two vector ops
#pragma unroll
        for (int i = 0; i < ET * KS * MTW * 2; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, PQKV_ENC_VALU_PER_MFMA, 0);
        }
      };
      if (!kTable || step_fast) body(TableFlag<true>{});
      else body(TableFlag<false>{});
      store_rot(acc, g);
      gpp = gp;
      gp = g;
    }
    // the last step: quantise, then store it and the one before
    const int b = k & 1;
    wait_mem();
    barrier();
    if (gpp >= 0) flush(gpp, b ^ 1);
    float r, inv;
    const bool step_fast = finish(gp, b ^ 1, b, r, inv);
    if (!kTable || step_fast) quantise(table_flag, TableFlag<true>{}, acc, b, r, inv);
    else quantise(table_flag, TableFlag<false>{}, acc, b, r, inv);
    barrier();
    flush(gp, b);
  };
  // Set-up: the first step's input copies and R's loads are in flight while
  // the centroid table is built (its barriers wait for LDS only).
  issue(blockIdx.x, 0);
  lds_barrier();
  build_cell_table(cb, NL, tid, cells, thr, ucell, &table_ok);
  split_r();
  if constexpr (QJL) {
    if (table_ok != 0) run_qjl(TableFlag<true>{});
    else run_qjl(TableFlag<false>{});
  } else {
    if (table_ok != 0) run(TableFlag<true>{});
    else run(TableFlag<false>{});
  }
}

hipError_t launch_encode_mfma(const EncodeArgs &a, float *rot_out, float *radius_out, int cus, hipStream_t s) {
  const bool qjl = a.qjl != nullptr || a.qjl_pages != nullptr;
  const int64_t n = a.n_outer * a.n_inner;
  const int eg = qjl ? 32 : kEG;
  const int64_t groups = (n + eg - 1) / eg;
  // each workgroup keeps its share of R in registers and builds its centroid
  // table once, so one resident round of workgroups loops over the steps
  int64_t grid = groups;
  if (grid > kEBlocksPerCU * (int64_t)cus) grid = kEBlocksPerCU * (int64_t)cus;
  if (grid < 1) grid = 1;
#define PQKV_EM(DD, BB, QQ) encode_mfma_kernel<DD, BB, QQ><<<(int)grid, kEW * 64, 0, s>>>(a, rot_out, radius_out)
#define PQKV_EMQ(DD, BB) \
  if (qjl) PQKV_EM(DD, BB, true); \
  else PQKV_EM(DD, BB, false)
  if (a.d == 128 && a.bits == 4) PQKV_EMQ(128, 4);
  else if (a.d == 128 && a.bits == 2) PQKV_EMQ(128, 2);
  else if (a.d == 64 && a.bits == 4) PQKV_EMQ(64, 4);
  else PQKV_EMQ(64, 2);
#undef PQKV_EMQ
#undef PQKV_EM
  return hipGetLastError();
}

}  // namespace pqkv
