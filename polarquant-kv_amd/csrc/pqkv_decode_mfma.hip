// Split-K decode attention on the matrix cores (gfx950 v_mfma_f32_16x16x32_f16)
// for block_pq4 keys and values.
//
// Same contract and workspace format as decode_split_kernel (pqkv_decode.hip):
// scores q_rot . c[idx] * r_k, online softmax in the exp2 domain, values
// sum_t w_t r_v,t c[vidx_t], per-split (max, sum, unnormalised output).
//
// Precision: the 2e-3 absolute output tolerance on outlier-channel caches
// needs fp32-grade products, so every fp32 operand x is split into
//   x_hi = fp16(x),  x_lo = fp16((x - x_hi) * 2^11)
// (x_lo stays in the fp16 normal range, so no fp16 subnormals are involved):
//   x . y = x_hi.y_hi + 2^-11 (x_lo.y_hi + x_hi.y_lo)   (+ O(2^-22)).
// The GEMM's k index runs over (element, part): B holds (y_hi, y_lo) pairs,
// and with at most 8 query heads one 16-row A tile holds
//   rows 0-7  (heads): (x_hi, 0)         -> D[h]     = sum x_hi y_hi
//   rows 8-15 (heads): (x_lo, x_hi)      -> D[h + 8] = sum x_lo y_hi + x_hi y_lo
// so result[h] = D[h] + 2^-11 D[h + 8], one MFMA per 16 elements.
//
// Layouts (16x16x32 f16; verified on the device): A lane l holds row l%16,
// k = 8(l/16)+i; B lane l holds column l%16, k = 8(l/16)+i; D lane l holds
// rows 4(l/16)+i, column l%16. Below col = l%16, grp = l/16.
//   scores, transposed: S^T[token][col] = A(K codes) . B(q parts); a lane's
//     A row is one token, its 8 k values 4 coordinates x (hi, lo) = two packed
//     bytes, each read from a 256-entry table of (c_hi, c_lo, c_hi', c_lo').
//     The result sits in D with token rows 4grp+i and head column col, which
//     is exactly the A layout the value product needs for the softmax
//     weights: no transposition through LDS.
//   values: O[head row][coord] = A(p parts) . B(V codes); a lane's B column is
//     one coordinate, its 8 k values 4 tokens x (hi, lo): two tokens' nibbles
//     of that coordinate interleaved into one byte give both tokens' values
//     with the same kind of table read.
// Cross-lane steps use DPP row rotations and the gfx950 permlane16/32 swaps
// (VALU), not LDS permutes; LDS carries only the chunk tiles and the tables.
#include "pqkv_device.h"
#include "pqkv_launch.h"

namespace pqkv {

namespace {

constexpr int kMWaves = 4;
constexpr int kSub = 16;             // tokens per MFMA tile
constexpr int kChunk = 64;           // tokens per wave iteration
constexpr float kLoScale = 2048.0f;  // 2^11

__device__ __forceinline__ void split_hi_lo(float x, half_t *hi, half_t *lo) {
  const half_t h = (half_t)x;
  *hi = h;
  *lo = (half_t)__builtin_fmaf(x, kLoScale, -(float)h * kLoScale);
}

__device__ __forceinline__ uint32_t pack_h2(half_t a, half_t b) {
  half2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, v);
}

// byte b -> halfs (c_hi[b & 15], c_lo[b & 15], c_hi[b >> 4], c_lo[b >> 4])
__device__ __forceinline__ void build_lut_pairs(uint2 *lut, const float *cb, int tid) {
  if (tid < 256) {
    half_t h0, l0, h1, l1;
    split_hi_lo(cb[tid & 15], &h0, &l0);
    split_hi_lo(cb[tid >> 4], &h1, &l1);
    lut[tid] = make_uint2(pack_h2(h0, l0), pack_h2(h1, l1));
  }
}

__device__ __forceinline__ half8_t pack8(uint2 a, uint2 b) {
  typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
  u32x4v v = {a.x, a.y, b.x, b.y};
  return __builtin_bit_cast(half8_t, v);
}
__device__ __forceinline__ half8_t pack8u(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
  u32x4v v = {a, b, c, d};
  return __builtin_bit_cast(half8_t, v);
}

__device__ __forceinline__ float4_t mfma16(half8_t a, half8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Lane col of each 16-lane row receives lane (col + 8) % 16 (DPP row_ror:8).
__device__ __forceinline__ uint32_t row_ror8(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x128, 0xF, 0xF, false);
}
__device__ __forceinline__ float row_ror8f(float x) { return __builtin_bit_cast(float, row_ror8(__builtin_bit_cast(uint32_t, x))); }

// Combine the same lane position of the four 16-lane rows (gfx950 swaps).
__device__ __forceinline__ float rows_max(float x) {
  auto a = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x), false, false);
  x = fmaxf(__builtin_bit_cast(float, (uint32_t)a[0]), __builtin_bit_cast(float, (uint32_t)a[1]));
  auto b = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x), false, false);
  return fmaxf(__builtin_bit_cast(float, (uint32_t)b[0]), __builtin_bit_cast(float, (uint32_t)b[1]));
}
__device__ __forceinline__ float rows_sum(float x) {
  auto a = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x), false, false);
  x = __builtin_bit_cast(float, (uint32_t)a[0]) + __builtin_bit_cast(float, (uint32_t)a[1]);
  auto b = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x), false, false);
  return __builtin_bit_cast(float, (uint32_t)b[0]) + __builtin_bit_cast(float, (uint32_t)b[1]);
}

// Raw buffer over one (batch, head) stream: loads past `bytes` return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t stream_rsrc(const uint8_t *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 bld128(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) volatile u32x2 lds_u32x2;

// 8-byte LDS store the compiler neither merges nor turns into a flat store.
__device__ __forceinline__ void lds_store8(uint8_t *p, u32x2 v) { *(lds_u32x2 *)p = v; }

// One 64-token chunk of K and V as contiguous 16-byte pieces: lane l holds
// pieces l + 64 j.
template <int D>
struct ChunkRegs {
  static constexpr int kBytes = kChunk * vector_bytes(D, 4);  // per stream
  static constexpr int kPieces = kBytes / 16;
  static constexpr int kPerLane = (kPieces + 63) / 64;
  u32x4 k[kPerLane], v[kPerLane];
};

template <int D>
__device__ __forceinline__ void load_chunk(ChunkRegs<D> &c, __amdgpu_buffer_rsrc_t kr, __amdgpu_buffer_rsrc_t vr,
                                           int t0, int lane) {
  using CR = ChunkRegs<D>;
  const int base = t0 * vector_bytes(D, 4);
#pragma unroll
  for (int j = 0; j < CR::kPerLane; ++j) {
    const int piece = lane + 64 * j;
    if (j < CR::kPerLane - 1 || piece < CR::kPieces) {
      c.k[j] = bld128(kr, base + 16 * piece);
      c.v[j] = bld128(vr, base + 16 * piece);
    }
  }
}

// LDS tiles keep the HBM byte layout. 8-byte stores run at the full LDS rate
// (16-byte ones at half); volatile keeps the compiler from merging them.
template <int D>
__device__ __forceinline__ void stage_chunk(const ChunkRegs<D> &c, uint8_t *ktile, uint8_t *vtile, int lane) {
  using CR = ChunkRegs<D>;
#pragma unroll
  for (int j = 0; j < CR::kPerLane; ++j) {
    const int piece = lane + 64 * j;
    if (j < CR::kPerLane - 1 || piece < CR::kPieces) {
      lds_store8(ktile + 16 * piece, c.k[j].xy);
      lds_store8(ktile + 16 * piece + 8, c.k[j].zw);
      lds_store8(vtile + 16 * piece, c.v[j].xy);
      lds_store8(vtile + 16 * piece + 8, c.v[j].zw);
    }
  }
}

// qs dword holding coordinates 32m + 8*sub .. +7 (sub = 0..3) of one vector:
// byte offset 18m + 2 + 4 sub, misaligned by two bytes when m is even.
__device__ __forceinline__ uint32_t qs_dword(const uint8_t *vec, int m, int sub) {
  const int off = m * kPq4BlockBytes + 2 + 4 * sub;
  if (m & 1) return *(const uint32_t *)(vec + off);
  const uint32_t *p = (const uint32_t *)(vec + off - 2);
  return align_bytes(p[1], p[0], 2);
}

}  // namespace

template <int D, int G>
__global__ void __launch_bounds__(256, kMfmaBlocksPerCU) decode_mfma_kernel(const DecodeArgs a) {
  constexpr int VB = vector_bytes(D, 4);
  constexpr int KK = D / 16;     // score MFMAs per 16-token tile
  constexpr int NB = D / 16;     // value n-tiles
  constexpr int NSUB = kChunk / kSub;
  constexpr int TILE = kChunk * VB;

  // One LDS block with the tables first, so their addresses fit the 16-bit
  // immediate offset of ds_read (the whole block is 80 KB). Per wave: two
  // chunk buffers (the chunk being finished and the next one), each a K and a
  // V tile plus their gathered radii.
  struct Smem {
    uint2 lut_k[256], lut_v[256];
    float red_m[kMWaves][8], red_l[kMWaves][8];
    uint16_t rad[kMWaves][2][2][kChunk];
    __attribute__((aligned(16))) uint8_t tiles[kMWaves][2][2][TILE + 16];
  };
  __shared__ Smem sm;
  uint2 *lut_k = sm.lut_k, *lut_v = sm.lut_v;
  auto &tiles = sm.tiles;
  auto &rad = sm.rad;
  auto &red_m = sm.red_m;
  auto &red_l = sm.red_l;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int split = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / a.n_heads, hi_ = bh - b * a.n_heads;
  const int h = a.listed ? a.heads[hi_] : hi_;
  const int t_begin = split * a.tokens_per_split;
  const int t_end = min(a.S, t_begin + a.tokens_per_split);
  const uint8_t *kstream, *vstream;
  if (a.listed) {
    kstream = a.k_cache + b * a.k_batch_stride + a.k_head_off[hi_];
    vstream = a.v_cache + b * a.v_batch_stride + a.v_head_off[hi_];
  } else {
    kstream = a.k_cache + b * a.k_batch_stride + h * a.k_head_stride;
    vstream = a.v_cache + b * a.v_batch_stride + h * a.v_head_stride;
  }
  const uint32_t valid_bytes = (uint32_t)a.S * (uint32_t)VB;
  const __amdgpu_buffer_rsrc_t kres = stream_rsrc(kstream, valid_bytes);
  const __amdgpu_buffer_rsrc_t vres = stream_rsrc(vstream, valid_bytes);

  build_lut_pairs(lut_k, a.k_cb + h * a.cb_head_stride, tid);
  build_lut_pairs(lut_v, a.v_cb + h * a.cb_head_stride, tid);

  // q as the B operand of the score product: column col = (head col & 7,
  // part col >> 3); step kk, k = 8grp + i covers coordinate
  // 32(kk/2) + 8grp + 4(kk%2) + i/2, part i%2:
  //   col < 8 : (q_hi, 0)        col >= 8 : (q_lo, q_hi)
  const int qh = col & 7;
  const bool qlo = col >= 8;
  const float qmask = qh < G ? 1.0f : 0.0f;
  const float *qrow = a.q + (int64_t)(b * a.Hq + h * G + (qh < G ? qh : 0)) * D;
  half8_t qb[KK];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      half_t vh, vl;
      split_hi_lo(qrow[32 * (kk >> 1) + 8 * grp + 4 * (kk & 1) + j] * qmask, &vh, &vl);
      qb[kk][2 * j] = qlo ? vl : vh;
      qb[kk][2 * j + 1] = qlo ? vh : (half_t)0.0f;
    }
  }

  // Running softmax state: lanes with col < 8 own head col (replicated over
  // the four rows).
  float m_run = -INFINITY, l_run = 0.0f;
  float4_t oacc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) oacc[nb] = (float4_t){0.f, 0.f, 0.f, 0.f};

  // Value side: lane's coordinate group (qs dword) and, for D = 64, parity.
  const int vw = D == 128 ? col : (col & 7);
  const int vpar = D == 128 ? 0 : (col >> 3);
  const int vob = (vw >> 2) * kPq4BlockBytes + 2 + 4 * (vw & 3);
  const int vob_al = vob & ~3, vsh = vob & 3;

  ChunkRegs<D> cr_;
  __syncthreads();

  // Stage a chunk (held in registers) into buffer `buf` and gather its radii.
  auto stage = [&](int buf) {
    stage_chunk<D>(cr_, tiles[wave][buf][0], tiles[wave][buf][1], lane);
    rad[wave][buf][0][lane] = *(const uint16_t *)(tiles[wave][buf][0] + lane * VB);
    rad[wave][buf][1][lane] = *(const uint16_t *)(tiles[wave][buf][1] + lane * VB);
  };
  // Scores of the chunk in buffer `buf`: S^T[token][col] per 16-token tile.
  auto scores = [&](int buf, float4_t (&sacc)[NSUB]) {
    const uint8_t *ktile = tiles[wave][buf][0];
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int st = 0; st < NSUB; ++st) {
      const uint8_t *kv = ktile + (kSub * st + col) * VB;
      uint2 kt[KK][2];
#pragma unroll
      for (int m = 0; m < KK / 2; ++m) {
        const uint32_t w = qs_dword(kv, m, grp);
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          kt[2 * m + e][0] = lut_k[(w >> (16 * e)) & 0xFF];
          kt[2 * m + e][1] = lut_k[(w >> (16 * e + 8)) & 0xFF];
        }
      }
      sacc[st] = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) sacc[st] = mfma16(pack8(kt[kk][0], kt[kk][1]), qb[kk], sacc[st]);
    }
    __builtin_amdgcn_s_setprio(0);
  };
  // Softmax update and value product of the chunk in buffer `buf` whose
  // scores are `sacc`; tokens >= ntok of the chunk are masked.
  auto finish = [&](int buf, const float4_t (&sacc)[NSUB], int ntok, bool partial) {
    const uint8_t *vtile = tiles[wave][buf][1];
    const uint16_t *rk_lds = rad[wave][buf][0], *rv_lds = rad[wave][buf][1];
    // s = D[t][h] + 2^-11 D[t][h + 8] for token 16st + 4grp + i, meaningful
    // in lanes col < G. Lanes of absent heads (q = 0) and the cross lanes
    // (col >= 8) carry finite values that only reach discarded output rows.
    float sv[NSUB][4];
#pragma unroll
    for (int st = 0; st < NSUB; ++st) {
      const uint2 rk4 = *(const uint2 *)&rk_lds[kSub * st + 4 * grp];
      const uint32_t rkw[2] = {rk4.x, rk4.y};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float cross = row_ror8f(sacc[st][i]);
        const float rk = half_bits_to_float(rkw[i >> 1] >> (16 * (i & 1)));
        sv[st][i] = __builtin_fmaf(cross, 1.0f / kLoScale, sacc[st][i]) * rk;
      }
    }
    if (partial) {
#pragma unroll
      for (int st = 0; st < NSUB; ++st)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (kSub * st + 4 * grp + i >= ntok) sv[st][i] = -INFINITY;
    }
    float cmax = sv[0][0];
#pragma unroll
    for (int st = 0; st < NSUB; ++st)
#pragma unroll
      for (int i = 0; i < 4; ++i) cmax = fmaxf(cmax, sv[st][i]);
    // token 0 of the chunk is valid, so after the row reduction every lane's
    // max is finite; the first chunk has m_run = -inf and alpha = 0.
    cmax = rows_max(cmax);
    const float mnew = fmaxf(m_run, cmax);
    const float alpha = __builtin_amdgcn_exp2f(m_run - mnew);
    m_run = mnew;
    // rescale the running output: lane (col, grp) holds rows 4grp + i, i.e.
    // head 4(grp & 1) + i (hi part for grp < 2, cross part for grp >= 2);
    // alpha of head hh sits in lane hh. Skipped (wave-uniform) when no head's
    // maximum moved, the common case once the first chunks are in.
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) & 0xFFull) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // lane gather (a select between two read-lanes becomes a scratch
        // array indexed by the lane group)
        const float f = __builtin_bit_cast(
            float, __builtin_amdgcn_ds_bpermute(4 * (4 * (grp & 1) + i), __builtin_bit_cast(int, alpha)));
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) oacc[nb][i] *= f;
      }
    }
    // values, one 16-token k-block per MFMA step
    float psum = 0.0f;
#pragma unroll
    for (int kb = 0; kb < NSUB; ++kb) {
      // value-side entries: two tokens' nibbles of the lane's coordinate
      // interleaved into one byte (token pairs (0,1) and (2,3))
      uint32_t wv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t *pv = (const uint32_t *)(vtile + (kSub * kb + 4 * grp + e) * VB + vob_al);
        wv[e] = align_bytes(pv[1], pv[0], vsh);
      }
      // byte k of x = even coordinate 2k of both tokens, of y = odd 2k + 1
      const uint32_t x01 = (wv[0] & 0x0F0F0F0Fu) | ((wv[1] << 4) & 0xF0F0F0F0u);
      const uint32_t y01 = ((wv[0] >> 4) & 0x0F0F0F0Fu) | (wv[1] & 0xF0F0F0F0u);
      const uint32_t x23 = (wv[2] & 0x0F0F0F0Fu) | ((wv[3] << 4) & 0xF0F0F0F0u);
      const uint32_t y23 = ((wv[2] >> 4) & 0x0F0F0F0Fu) | (wv[3] & 0xF0F0F0F0u);
      uint2 vt[NB][2];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        // D = 128: n-tile nb is nibble nb of dword col (coordinate 8*col + nb).
        // D = 64: n-tile nb is coordinate 8*(col & 7) + 2*nb + (col >> 3).
        const int par = D == 128 ? (nb & 1) : vpar;
        const int byte = D == 128 ? (nb >> 1) : nb;
        vt[nb][0] = lut_v[((par ? y01 : x01) >> (8 * byte)) & 0xFF];
        vt[nb][1] = lut_v[((par ? y23 : x23) >> (8 * byte)) & 0xFF];
      }
      // weights p * r_v in the A layout: col < 8 -> (p_hi, 0), col >= 8 ->
      // (p_lo, p_hi) of head col - 8, taken from lane col - 8.
      const uint2 rv4 = *(const uint2 *)&rv_lds[kSub * kb + 4 * grp];
      const uint32_t rvw[2] = {rv4.x, rv4.y};
      uint32_t pa[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = __builtin_amdgcn_exp2f(sv[kb][i] - mnew);
        psum += p;
        half_t ph, pl;
        split_hi_lo(p * half_bits_to_float(rvw[i >> 1] >> (16 * (i & 1))), &ph, &pl);
        const uint32_t top = pack_h2(ph, (half_t)0.0f);
        const uint32_t bot = row_ror8(pack_h2(pl, ph));
        pa[i] = col < 8 ? top : bot;
      }
      const half8_t pav = pack8u(pa[0], pa[1], pa[2], pa[3]);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) oacc[nb] = mfma16(pav, pack8(vt[nb][0], vt[nb][1]), oacc[nb]);
    }
    l_run = l_run * alpha + psum;
  };

  // The wave's chunks start at first + i * kStep. Iteration i finishes chunk
  // i (softmax + values) and computes the scores of chunk i + 1 in the same
  // straight-line block, so each one's LDS latency hides behind the other's
  // work; the chunk i + 2 codes are in flight meanwhile. Only the last chunk
  // can be partial; it is finished after the loop.
  constexpr int kStep = kMWaves * kChunk;
  const int first = t_begin + wave * kChunk;
  const int nch = first < t_end ? (t_end - first + kStep - 1) / kStep : 0;
  if (nch > 0) {
    load_chunk<D>(cr_, kres, vres, first, lane);
    stage(0);
    if (nch > 1) load_chunk<D>(cr_, kres, vres, first + kStep, lane);
    float4_t sacc[NSUB];
    scores(0, sacc);
    for (int i = 0; i + 1 < nch; ++i) {
      const int nxt = (i + 1) & 1;
      stage(nxt);
      // chunk i + 2 (a repeat of the last chunk past the end: an L2 hit)
      const int tl = first + min(i + 2, nch - 1) * kStep;
      load_chunk<D>(cr_, kres, vres, tl, lane);
      float4_t snext[NSUB];
      scores(nxt, snext);
      finish(i & 1, sacc, kChunk, false);
#pragma unroll
      for (int st = 0; st < NSUB; ++st) sacc[st] = snext[st];
    }
    const int tlast = first + (nch - 1) * kStep;
    finish((nch - 1) & 1, sacc, min(kChunk, t_end - tlast), true);
  }

  // ---------------- per-wave results ----------------
  // l: sum over the four rows of lane col; m is already row-uniform.
  l_run = rows_sum(l_run);
  if (lane < G) {
    red_m[wave][lane] = m_run;
    red_l[wave][lane] = l_run;
  }
  // O[head][coord] = D[head] + 2^-11 D[head + 8]: rows 8-15 sit 32 lanes up.
  float *red_o = (float *)tiles[wave][0];  // this wave's tile is free now
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // (once per block: a plain cross-lane read; hipcc 7.2 picks the wrong
      // source register for permlane32_swap on extracted vector elements)
      const float cross = shfl_xor_f(oacc[nb][i], 32);
      const int head = 4 * grp + i;
      if (grp < 2 && head < G) {
        const int coord = D == 128 ? 8 * col + nb : 8 * (col & 7) + 2 * nb + (col >> 3);
        red_o[head * D + coord] = __builtin_fmaf(cross, 1.0f / kLoScale, oacc[nb][i]);
      }
    }
  __syncthreads();
  for (int i = tid; i < G * D; i += 256) {
    const int hh = i / D, c = i - hh * D;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kMWaves; ++w) mx = fmaxf(mx, red_m[w][hh]);
    float L = 0.0f, O = 0.0f;
#pragma unroll
    for (int w = 0; w < kMWaves; ++w) {
      const float sc = red_m[w][hh] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(red_m[w][hh] - mx);
      L += red_l[w][hh] * sc;
      O += ((const float *)tiles[w][0])[hh * D + c] * sc;
    }
    float *dst = a.part + (((int64_t)(b * a.Hq + h * G + hh) * a.splits) + split) * (D + 2);
    if (c == 0) {
      dst[0] = mx;
      dst[1] = L;
    }
    dst[2 + c] = O;
  }
}

template <int D>
static void launch_dm(const DecodeArgs &a, int G, hipStream_t s) {
  dim3 grid(a.splits, a.B * a.n_heads);
  switch (G) {
    case 1: decode_mfma_kernel<D, 1><<<grid, 256, 0, s>>>(a); break;
    case 2: decode_mfma_kernel<D, 2><<<grid, 256, 0, s>>>(a); break;
    case 3: decode_mfma_kernel<D, 3><<<grid, 256, 0, s>>>(a); break;
    case 4: decode_mfma_kernel<D, 4><<<grid, 256, 0, s>>>(a); break;
    case 5: decode_mfma_kernel<D, 5><<<grid, 256, 0, s>>>(a); break;
    case 6: decode_mfma_kernel<D, 6><<<grid, 256, 0, s>>>(a); break;
    case 7: decode_mfma_kernel<D, 7><<<grid, 256, 0, s>>>(a); break;
    default: decode_mfma_kernel<D, 8><<<grid, 256, 0, s>>>(a); break;
  }
}

hipError_t launch_decode_mfma(const DecodeArgs &a, hipStream_t s) {
  const int G = a.Hq / a.Hkv;
  if (a.d == 128) launch_dm<128>(a, G, s);
  else launch_dm<64>(a, G, s);
  return hipGetLastError();
}

}  // namespace pqkv
