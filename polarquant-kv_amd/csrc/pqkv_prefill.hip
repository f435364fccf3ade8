// Chunked-prefill attention on the matrix cores (gfx950 v_mfma_f32_16x16x32_f16)
// over block_pq4 / block_pq2 keys and values, optionally with the QJL sign
// correction on the keys.
//
// Sq query tokens per sequence, at absolute positions q_start.., attend to a
// cache that already holds them (append-then-attend). With causal set, query
// i sees cache positions <= q_start + i.
//
// Work split: one workgroup = 8 waves = 256 query rows of one (batch, kv-head),
// a row being (query token, head of the group): row r -> token r / G, head
// r % G. Each wave owns 32 rows (two 16-row tiles); with QJL 16 rows (one
// tile, 128 rows per workgroup), which leaves registers for the projection
// operands. The KV cache is walked in
// 64-token tiles. Each tile is decoded once per workgroup into LDS, as fp16
// planes in the exact order the MFMA operands want, so that every operand
// read is a conflict-free run of 8-byte loads. Tiles are double-buffered.
// The waves run a two-group ping-pong schedule (matrix stage against softmax
// and decode stage, one group a stage behind the other), described at the
// main loop.
//
// Scores are computed transposed, S^T[token][row] = K^ . Q^T: K^ (16 tokens x
// 32 coordinates) is the A operand and the rotated queries the B operand, so
// the result lands in the D layout with tokens on rows and query rows on
// columns. That is the A layout of the P . V^ product, so the softmax weights
// never leave the lanes (the same trick as the decode kernel).
//
// 2-bit codes: a nibble holds two codes, so 16-entry tables give the same
// operand pairs as the 4-bit byte tables.
// QJL: s += [e != 0] sum_i (2 sign_i - 1) pq_i, pq = P_rot q_rot / m, a
// second product per score tile: A = the signs as +-1 halves (a 16-entry
// table maps 4 sign bits to 4 halves; a key whose sketch is all ones, which
// is what a zero residual e gives, reads a zero entry: the reference's guard,
// python/polarquant_kv/qjl.py:50-51),
// B = pq hi / lo. The key radius then scales the code product before the
// sign product is added (in the matrix stage instead of the softmax).
//
// Precision: every fp32 operand x is split as x_hi = fp16(x),
// x_lo = fp16(x - x_hi) (fp16 subnormals included, which the f16 MFMA keeps),
// and each product is hi.hi + hi.lo + lo.hi in one fp32 accumulator: three
// MFMAs per tile product, relative error ~2^-21 per term while x_lo is a
// normal number (|x| >= 2^-3). The codebook planes and the queries are
// therefore split at 2^6 times their value (kPlaneScale: centroids of
// 0.003 .. 0.33 and queries down to ~0.002 keep normal lo parts); the exact
// power-of-two factors come back out through the key radii (/ 2^12) and the
// final normalisation (/ 2^6).
#include "pqkv_device.h"
#include "pqkv_launch.h"

namespace pqkv {

namespace {

constexpr int kPW = 8;                    // waves per workgroup
constexpr int kPRowsWave = 32;            // query rows per wave
constexpr int kPT = 64;                   // kv tokens per tile
constexpr int kSegBytes = 64 * 8;         // one operand segment: 64 lanes x 8 bytes
constexpr float kPlaneScale = kPrefillPlaneScale;              // codebook planes and queries, x 2^6
constexpr float kScoreUnscale = 1.0f / (kPlaneScale * kPlaneScale);

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) u32x2 lds_u32x2;
typedef __attribute__((address_space(3))) const u32x2 lds_cu32x2;

__device__ __forceinline__ void lds_put8(uint8_t *p, uint32_t a, uint32_t b) { *(lds_u32x2 *)p = (u32x2){a, b}; }
__device__ __forceinline__ u32x2 lds_get8(const uint8_t *p) { return *(lds_cu32x2 *)p; }

__device__ __forceinline__ void split2(float x, half_t *hi, half_t *lo) {
  const half_t h = (half_t)x;
  *hi = h;
  *lo = (half_t)(x - (float)h);
}

__device__ __forceinline__ uint32_t pack_h2(half_t a, half_t b) {
  half2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ half8_t pack8u(u32x2 a, u32x2 b) {
  typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
  u32x4v v = {a.x, a.y, b.x, b.y};
  return __builtin_bit_cast(half8_t, v);
}

__device__ __forceinline__ float4_t mfma16(half8_t a, half8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

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

// Value of lane `row` (0..15) for output row 4 grp + i (v is the same in
// the four lanes of a column): one lane gather per i.
__device__ __forceinline__ void per_row(float v, int grp, float (&f)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
    f[i] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(4 * (4 * grp + i), __builtin_bit_cast(int, v)));
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t stream_rsrc(const uint8_t *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint32_t bld32(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ uint32_t bld16(__amdgpu_buffer_rsrc_t r, int off) {
  return (uint32_t)__builtin_bit_cast(uint16_t, __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0));
}

}  // namespace

template <int D>
struct PrefillTile {
  static constexpr int KS = D / 32;              // k-steps of the score product
  static constexpr int NB = D / 16;              // n-tiles of the value product
  static constexpr int KSEG = 4 * KS * 2 * 2;    // K segments: (tt, ks, plane, half)
  static constexpr int VSEG = NB * 2 * 2 * 2;    // V segments: (nb, kk, plane, half)
  static constexpr int BYTES = (KSEG + VSEG) * kSegBytes;
  static constexpr int KITEMS = kPT * (D / 8);   // (token, 8-coordinate group)
  static constexpr int VITEMS = (kPT / 4) * (D / 8);  // (4-token group, 8-coordinate group)
  __device__ static int kseg(int tt, int ks, int plane, int h) { return ((tt * KS + ks) * 2 + plane) * 2 + h; }
  __device__ static int vseg(int nb, int kk, int plane, int h) { return KSEG + ((nb * 2 + kk) * 2 + plane) * 2 + h; }
};

// Raw block bytes of one 64-token tile of one stream, staged in LDS by
// buffer-to-LDS loads (1 KB per wave instruction) so that no code registers
// stay live across the schedule's stages. Sized for 4-bit codes, the larger.
template <int D>
struct RawTile {
  static constexpr int kBytes = kPT * vector_bytes(D, 4);
  static constexpr int kPieces = (kBytes + 1023) / 1024;
  static constexpr int kAlloc = kPieces * 1024;
};

// One group's four waves copy tile t0 of a stream of VB-byte vectors into
// `raw`; bytes past the stream's end arrive as zeros.
template <int VB>
__device__ __forceinline__ void dma_raw(__amdgpu_buffer_rsrc_t r, uint8_t *raw, int t0, int gw, int lane) {
  constexpr int kPieces = (kPT * VB + 1023) / 1024;
#pragma unroll
  for (int j = 0; j < (kPieces + 3) / 4; ++j) {
    const int p = gw + 4 * j;
    if (p < kPieces)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)(raw + 1024 * p), 16,
                                               t0 * VB + 1024 * p + 16 * lane, 0, 0, 0);
  }
}

// The codes of coordinates 8 g8 .. 8 g8 + 7 of tile vector t in LDS: a dword
// of 8 nibbles (4-bit, block g8 / 4, qs bytes 4 (g8 % 4) ..) or a half
// dword of 8 crumbs (2-bit, qs bytes 2 (g8 % 4) ..).
template <int D, int BITS>
__device__ __forceinline__ uint32_t raw_code_word(const uint8_t *raw, int t, int g8) {
  constexpr int VB = vector_bytes(D, BITS);
  if constexpr (BITS == 4) {
    const int off = t * VB + (g8 >> 2) * kPq4BlockBytes + 2 + 4 * (g8 & 3);
    const uint32_t *p = (const uint32_t *)(raw + (off & ~3));
    return align_bytes(p[1], p[0], off & 3);
  } else {
    const int off = t * VB + (g8 >> 2) * kPq2BlockBytes + 2 + 2 * (g8 & 3);   // even
    return *(const uint16_t *)(raw + off);
  }
}

// Table index of code unit u (two coordinates: 2u, 2u + 1) of a code word.
template <int BITS>
__device__ __forceinline__ uint32_t code_unit(uint32_t w, int u) {
  return BITS == 4 ? (w >> (8 * u)) & 0xFF : (w >> (4 * u)) & 0xF;
}

// The thread index passed through an opaque move: the decode addresses
// derived from it are then recomputed in each stage (a few VALU operations)
// instead of being hoisted out of the tile loop and spilled.
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// K items: item i is operand lane L = i % 64 of segment pair (tt, ks) =
// (i / 64) / KS, (i / 64) % KS: token 16 tt + L % 16, coordinates
// 32 ks + 8 (L / 16) .. + 7. A wave's items are one (tt, ks) with L = its
// lane, so its LDS writes are contiguous runs.
template <int D>
__device__ __forceinline__ void k_item(int item, int &t, int &g8) {
  constexpr int KS = PrefillTile<D>::KS;
  const int tk = item >> 6, L = item & 63;
  t = 16 * (tk / KS) + (L & 15);
  g8 = 4 * (tk % KS) + (L >> 4);
}

// Decode a staged K tile into LDS: K^ hi / lo planes in operand order, and
// fp32 key radii. Run by group 0 (gtid 0..255).
template <int D, int KB>
__device__ __forceinline__ void decode_k(const uint8_t *raw, uint8_t *tile, float *rad, const uint2 *lut_k,
                                         int gtid) {
  using PT = PrefillTile<D>;
  constexpr int VB = vector_bytes(D, KB);
  constexpr int KPER = PT::KITEMS / (kPW / 2 * 64);  // 4 (d = 128) or 2
  gtid = opaque(gtid);
#pragma unroll
  for (int u = 0; u < KPER; ++u) {
    int t, g8;
    k_item<D>(gtid + (kPW / 2) * 64 * u, t, g8);
    const int lane = 16 * (g8 & 3) + (t & 15);  // = the writing thread's lane
    const uint32_t w = raw_code_word<D, KB>(raw, t, g8);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      // coordinates 8 g8 + 4h .. +3: code units 2h, 2h + 1 of w
      const uint2 a = lut_k[code_unit<KB>(w, 2 * h)], b = lut_k[code_unit<KB>(w, 2 * h + 1)];
      lds_put8(tile + PT::kseg(t >> 4, g8 >> 2, 0, h) * kSegBytes + lane * 8, a.x, b.x);
      lds_put8(tile + PT::kseg(t >> 4, g8 >> 2, 1, h) * kSegBytes + lane * 8, a.y, b.y);
    }
  }
  // key radii carry the 2^-12 that undoes the plane and query scaling
  if (gtid < kPT) rad[gtid] = half_bits_to_float(*(const uint16_t *)(raw + gtid * VB)) * kScoreUnscale;
}

// Decode a staged V tile: V^ hi / lo planes in operand order, fp32 value
// radii. Run by group 1 (gtid 0..255).
template <int D, int VBITS>
__device__ __forceinline__ void decode_v(const uint8_t *raw, uint8_t *tile, float *rad, const uint2 *lut_v,
                                         int gtid) {
  using PT = PrefillTile<D>;
  constexpr int VB = vector_bytes(D, VBITS);
  gtid = opaque(gtid);
  if (gtid < PT::VITEMS) {
    const int q4 = gtid / (D / 8), g8 = gtid % (D / 8);
    const int tt = q4 >> 2, kk = tt >> 1, h = tt & 1, grp = q4 & 3;
    uint32_t c[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) c[j] = raw_code_word<D, VBITS>(raw, 4 * q4 + j, g8);
    // token pairs (0,1), (2,3): code unit k of x = coordinate 2k of both
    // tokens, of y = 2k + 1 (bytes of nibbles, or nibbles of crumbs)
    uint32_t x01, y01, x23, y23;
    if constexpr (VBITS == 4) {
      x01 = (c[0] & 0x0F0F0F0Fu) | ((c[1] << 4) & 0xF0F0F0F0u);
      y01 = ((c[0] >> 4) & 0x0F0F0F0Fu) | (c[1] & 0xF0F0F0F0u);
      x23 = (c[2] & 0x0F0F0F0Fu) | ((c[3] << 4) & 0xF0F0F0F0u);
      y23 = ((c[2] >> 4) & 0x0F0F0F0Fu) | (c[3] & 0xF0F0F0F0u);
    } else {
      x01 = (c[0] & 0x3333u) | ((c[1] << 2) & 0xCCCCu);
      y01 = ((c[0] >> 2) & 0x3333u) | (c[1] & 0xCCCCu);
      x23 = (c[2] & 0x3333u) | ((c[3] << 2) & 0xCCCCu);
      y23 = ((c[2] >> 2) & 0x3333u) | (c[3] & 0xCCCCu);
    }
    // Coordinate order rotated by g8 / 2: the 64 writes of one step then
    // cover 32 bank pairs (two per pair, the minimum for 512 bytes) instead
    // of sharing four.
#pragma unroll
    for (int step = 0; step < 8; ++step) {
      const int e = (step + (g8 >> 1)) & 7;
      const int dcoord = 8 * g8 + e;
      const int k = e >> 1;
      const uint32_t s01 = (e & 1) ? y01 : x01, s23 = (e & 1) ? y23 : x23;
      const uint2 a = lut_v[code_unit<VBITS>(s01, k)], b = lut_v[code_unit<VBITS>(s23, k)];
      const int lane = 16 * grp + (dcoord & 15);
      lds_put8(tile + PT::vseg(dcoord >> 4, kk, 0, h) * kSegBytes + lane * 8, a.x, b.x);
      lds_put8(tile + PT::vseg(dcoord >> 4, kk, 1, h) * kSegBytes + lane * 8, a.y, b.y);
    }
  }
  if (gtid < kPT) rad[kPT + gtid] = half_bits_to_float(*(const uint16_t *)(raw + gtid * VB));
}

template <int D, int KB, int VBITS, bool QJL>
__global__ void __launch_bounds__(kPW * 64, 1) prefill_mfma_kernel(const PrefillArgs a) {
  using PT = PrefillTile<D>;
  constexpr int KS = PT::KS, NB = PT::NB;
  constexpr int RT = QJL ? 1 : 2;                     // 16-row tiles per wave
  constexpr int VBK = vector_bytes(D, KB), VBV = vector_bytes(D, VBITS);
  constexpr int SGB = D / 8;                          // sign bytes per key (m = D)
  __shared__ uint2 lut_k[256], lut_v[256];
  __shared__ __attribute__((aligned(16))) uint8_t tiles[2][PT::BYTES];
  __shared__ __attribute__((aligned(16))) float rads[2][2 * kPT];  // [buf][k radii | v radii]
  // raw codes of the tiles being staged: group 0's stream K, group 1's V
  __shared__ __attribute__((aligned(16))) uint8_t raw[2][2][RawTile<D>::kAlloc];  // [group][buf]
  // QJL: raw sign bytes of tiles it % 3 (read in both groups' X(it), so a
  // third buffer keeps tile it + 2's copy off them) and the sign table
  // (entries 16..31 are zero: keys of zero radius get no correction)
  __shared__ __attribute__((aligned(16))) uint8_t raw_s[QJL ? 3 : 1][QJL ? kPT * SGB : 16];
  __shared__ uint2 lut_s[QJL ? 32 : 1];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;
  // Two groups of four waves; wave w and w + 4 share a SIMD.
  const int group = __builtin_amdgcn_readfirstlane(wave) >= kPW / 2 ? 1 : 0;  // wave-uniform
  const int gtid = tid - group * (kPW / 2) * 64;
  const int gw = __builtin_amdgcn_readfirstlane(wave) - group * (kPW / 2);
  const int G = a.G;
  const int qtile = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / a.n_heads, hl = bh - b * a.n_heads;
  const int h = a.listed ? a.heads[hl] : hl;
  const int q0 = qtile * a.qt;                       // first query token of the block
  const int q_last = min(a.Sq, q0 + a.qt) - 1;       // last valid query token
  const int kv_end = a.causal ? min(a.S, a.q_start + q_last + 1) : a.S;

  const uint8_t *kstream, *vstream;
  if (a.listed) {
    kstream = a.k_cache + b * a.k_batch_stride + a.k_head_off[hl];
    vstream = a.v_cache + b * a.v_batch_stride + a.v_head_off[hl];
  } else {
    kstream = a.k_cache + b * a.k_batch_stride + h * a.k_head_stride;
    vstream = a.v_cache + b * a.v_batch_stride + h * a.v_head_stride;
  }
  const __amdgpu_buffer_rsrc_t kres = stream_rsrc(kstream, (uint32_t)a.S * (uint32_t)VBK);
  const __amdgpu_buffer_rsrc_t vres = stream_rsrc(vstream, (uint32_t)a.S * (uint32_t)VBV);
  __amdgpu_buffer_rsrc_t sres = kres;
  if constexpr (QJL)
    sres = stream_rsrc(a.qjl + ((int64_t)(b * a.Hkv + h) * a.S_max) * SGB, (uint32_t)a.S * (uint32_t)SGB);

  // code unit (a byte of two 4-bit codes, a nibble of two 2-bit codes) ->
  // (c_hi, c_hi' | c_lo, c_lo') of its two codes
  auto build_lut = [&](uint2 *lut, const float *cb, int bits) {
    const int n = bits == 4 ? 256 : 16, sh = bits == 4 ? 4 : 2, mask = bits == 4 ? 15 : 3;
    if (tid < n) {
      half_t h0, l0, h1, l1;
      split2(cb[tid & mask] * kPlaneScale, &h0, &l0);
      split2(cb[tid >> sh] * kPlaneScale, &h1, &l1);
      lut[tid] = make_uint2(pack_h2(h0, h1), pack_h2(l0, l1));
    }
  };
  build_lut(lut_k, a.k_cb + h * a.cb_head_stride, KB);
  build_lut(lut_v, a.v_cb + h * a.cb_head_stride, VBITS);
  if constexpr (QJL) {
    if (tid < 32) {
      uint32_t hv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) hv[j] = tid >= 16 ? 0u : ((tid >> j) & 1) ? 0x3C00u : 0xBC00u;  // +-1.0 fp16
      lut_s[tid] = make_uint2(hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16));
    }
  }

  // Queries as the B operand: column col = row 16 RT wave + 16 rt + col;
  // step ks, k = 8 grp + i covers coordinate 32 ks + 8 grp + i. With QJL the
  // projections pq = P_rot q_rot / m the same way (projection 32 ks + 8 grp + i).
  half8_t qh[RT][KS], ql[RT][KS];
  half8_t pqh[QJL ? RT : 1][QJL ? KS : 1], pql[QJL ? RT : 1][QJL ? KS : 1];
  int row_pos[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int row = 16 * RT * wave + 16 * rt + col;
    const int tok = q0 + row / G, head = row % G;
    const bool row_ok = row < a.qt * G && tok < a.Sq;
    row_pos[rt] = a.q_start + tok;
    const int64_t qrow = ((int64_t)(b * a.Hq + h * G + head) * a.Sq) + (row_ok ? tok : 0);
    const float *qr = a.q + qrow * D;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        half_t vh, vl;
        split2(row_ok ? qr[32 * ks + 8 * grp + i] : 0.0f, &vh, &vl);
        qh[rt][ks][i] = vh;
        ql[rt][ks][i] = vl;
      }
    if constexpr (QJL) {
      const float *pr = a.pq + qrow * D;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          half_t vh, vl;
          split2(row_ok ? pr[32 * ks + 8 * grp + i] : 0.0f, &vh, &vl);
          pqh[rt][ks][i] = vh;
          pql[rt][ks][i] = vl;
        }
    }
  }

  float m_run[RT], l_run[RT];
  float4_t oacc[RT][NB];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    m_run[rt] = -INFINITY;
    l_run[rt] = 0.0f;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) oacc[rt][nb] = (float4_t){0.f, 0.f, 0.f, 0.f};
  }
  float4_t sacc[RT][4];                // scores of the tile between X and Y
  half8_t ph[RT][2], pl[RT][2];        // softmax weights between Y and the next X

  // ---- stage bodies ----
  // scores S^T[token][row] of tile it. The operands of step n + 1 are read
  // before step n's products (the fence keeps them there), so the LDS
  // latency hides behind six MFMAs.
  auto scores = [&](int it) {
    const uint8_t *tile = tiles[it & 1];
    auto kop = [&](int n, int plane) {
      const int tt = n / KS, ks = n % KS;
      return pack8u(lds_get8(tile + PT::kseg(tt, ks, plane, 0) * kSegBytes + lane * 8),
                    lds_get8(tile + PT::kseg(tt, ks, plane, 1) * kSegBytes + lane * 8));
    };
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) sacc[rt][tt] = (float4_t){0.f, 0.f, 0.f, 0.f};
    half8_t ah = kop(0, 0), al = kop(0, 1);
#pragma unroll
    for (int n = 0; n < 4 * KS; ++n) {
      const int tt = n / KS, ks = n % KS;
      half8_t ah_n = ah, al_n = al;
      if (n + 1 < 4 * KS) {
        ah_n = kop(n + 1, 0);
        al_n = kop(n + 1, 1);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        sacc[rt][tt] = mfma16(ah, qh[rt][ks], sacc[rt][tt]);
        sacc[rt][tt] = mfma16(al, qh[rt][ks], sacc[rt][tt]);
        sacc[rt][tt] = mfma16(ah, ql[rt][ks], sacc[rt][tt]);
      }
      ah = ah_n;
      al = al_n;
    }
    if constexpr (QJL) {
      // s = r_k (q . c) + [e != 0] sum_i (2 s_i - 1) pq_i: the radius
      // scaling moves here, then the sign products accumulate on top
      const float *rk = rads[it & 1];
      const uint8_t *sg = raw_s[it % 3];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const float4 r4 = *(const float4 *)&rk[16 * tt + 4 * grp];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          sacc[rt][tt][0] *= r4.x;
          sacc[rt][tt][1] *= r4.y;
          sacc[rt][tt][2] *= r4.z;
          sacc[rt][tt][3] *= r4.w;
        }
        // A: signs of token 16 tt + col, projections 32 ks + 8 grp .. + 7
        // (sign byte 4 ks + grp); the zero half of the table for an all-ones
        // sketch (the four lane groups' bytes of the token all 0xFF: bit col
        // of the ballot's four 16-lane slices ANDed)
        const int tok = 16 * tt + col;
        uint32_t sb[KS];
        uint32_t all = 0xFFu;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          sb[ks] = sg[tok * SGB + 4 * ks + grp];
          all &= sb[ks];
        }
        const uint64_t bal = __builtin_amdgcn_ballot_w64(all == 0xFFu);
        const uint32_t ones = (uint32_t)(bal & (bal >> 16) & (bal >> 32) & (bal >> 48));
        const int zoff = ((ones >> col) & 1u) ? 16 : 0;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const uint32_t byte = sb[ks];
          const uint2 lo = lut_s[zoff + (byte & 15)], hi = lut_s[zoff + (byte >> 4)];
          const half8_t as = pack8u((u32x2){lo.x, lo.y}, (u32x2){hi.x, hi.y});
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) {
            sacc[rt][tt] = mfma16(as, pqh[rt][ks], sacc[rt][tt]);
            sacc[rt][tt] = mfma16(as, pql[rt][ks], sacc[rt][tt]);
          }
        }
      }
    }
  };
  // O[row][coord] += P . V^ of tile it, operands read one step ahead
  auto values = [&](int it) {
    const uint8_t *tile = tiles[it & 1];
    auto vop = [&](int n, int plane) {
      const int nb = n >> 1, kk = n & 1;
      return pack8u(lds_get8(tile + PT::vseg(nb, kk, plane, 0) * kSegBytes + lane * 8),
                    lds_get8(tile + PT::vseg(nb, kk, plane, 1) * kSegBytes + lane * 8));
    };
    half8_t bh = vop(0, 0), bl = vop(0, 1);
#pragma unroll
    for (int n = 0; n < 2 * NB; ++n) {
      const int nb = n >> 1, kk = n & 1;
      half8_t bh_n = bh, bl_n = bl;
      if (n + 1 < 2 * NB) {
        bh_n = vop(n + 1, 0);
        bl_n = vop(n + 1, 1);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        oacc[rt][nb] = mfma16(ph[rt][kk], bh, oacc[rt][nb]);
        oacc[rt][nb] = mfma16(ph[rt][kk], bl, oacc[rt][nb]);
        oacc[rt][nb] = mfma16(pl[rt][kk], bh, oacc[rt][nb]);
      }
      bh = bh_n;
      bl = bl_n;
    }
  };
  // online softmax of tile it's scores -> weights p * r_v as the A operand
  auto softmax = [&](int it) {
    const int t0 = it * kPT;
    const float *rk = rads[it & 1], *rv = rads[it & 1] + kPT;
    const bool need_mask = t0 + kPT > a.S || (a.causal && t0 + kPT - 1 > a.q_start + q0);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float s[4][4];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const float4 r4 = *(const float4 *)&rk[16 * tt + 4 * grp];
        const float rr[4] = {r4.x, r4.y, r4.z, r4.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) s[tt][i] = QJL ? sacc[rt][tt][i] : sacc[rt][tt][i] * rr[i];
      }
      if (need_mask) {
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int t = t0 + 16 * tt + 4 * grp + i;
            if (t >= a.S || (a.causal && t > row_pos[rt])) s[tt][i] = -INFINITY;
          }
      }
      float cmax = s[0][0];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) cmax = fmaxf(cmax, s[tt][i]);
      cmax = rows_max(cmax);
      // token 0 is valid for every row, so m_run is finite after the first tile
      const float mnew = fmaxf(m_run[rt], cmax);
      const float alpha = __builtin_amdgcn_exp2f(m_run[rt] - mnew);
      m_run[rt] = mnew;
      float psum = 0.0f;
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const float4 r4 = *(const float4 *)&rv[16 * tt + 4 * grp];
        const float rr[4] = {r4.x, r4.y, r4.z, r4.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = __builtin_amdgcn_exp2f(s[tt][i] - mnew);
          psum += p;
          half_t vh, vl;
          split2(p * rr[i], &vh, &vl);
          // A operand of the value product: k = 8 grp + i' <-> token tile
          // 2 kk + i' / 4, token 4 grp + i' % 4
          ph[rt][tt >> 1][4 * (tt & 1) + i] = vh;
          pl[rt][tt >> 1][4 * (tt & 1) + i] = vl;
        }
      }
      l_run[rt] = l_run[rt] * alpha + psum;
      // the running output holds tiles < it here (tile it's values come in
      // the next X stage), so the rescale applies now; skipped (wave-uniform)
      // when no row's maximum moved, the common case after the first tiles
      if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
        float f[4];
        per_row(alpha, grp, f);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int i = 0; i < 4; ++i) oacc[rt][nb][i] *= f[i];
      }
    }
  };

  // ---- ping-pong schedule ----
  // Each tile takes two stages per wave: X(it) = values of tile it - 1 and
  // scores of tile it (matrix work), Y(it) = softmax of tile it plus one half
  // of tile it + 1's table decode (VALU and LDS work). Group 1 runs one stage
  // behind group 0 with a block barrier after every stage, so the two waves
  // sharing a SIMD are always in opposite stages: one's MFMA bursts overlap
  // the other's softmax and decode.
  // Tile it lives in buffer it & 1. Group 0 decodes K(it + 1) in its Y(it)
  // (stage 2 it + 1), after both groups' last read of K(it - 1) (stage
  // 2 it - 1); group 1 decodes V(it + 1) in its Y(it) (stage 2 it + 2), after
  // group 1's values of tile it - 1 (stage 2 it + 1). Each is read from the
  // stage after its decode on, and radii follow their half.
  const int ntiles = (kv_end + kPT - 1) / kPT;
  uint8_t(&graw)[2][RawTile<D>::kAlloc] = raw[group];
  // The buffer tile t0 is copied from and t0's position in it: the whole
  // stream, or with paged caches (pages != null, a wave-uniform test) the
  // tile's page over its valid tokens; a 64-token tile lies in one page.
  const int64_t prow = (int64_t)(b * a.Hkv + h) * a.max_pages;
  auto tile_rsrc = [&](const uint8_t *const *pages, __amdgpu_buffer_rsrc_t whole, int t0, int vb, int &rel) {
    if (pages == nullptr) {
      rel = t0;
      return whole;
    }
    const int pg = t0 >> a.page_shift, p0 = pg << a.page_shift;
    rel = t0 - p0;
    return stream_rsrc(pages[prow + pg], (uint32_t)min(a.S - p0, 1 << a.page_shift) * (uint32_t)vb);
  };
  auto decode = [&](int it) {  // this group's half of tile it, from graw[it & 1]
    if (group == 0) decode_k<D, KB>(graw[it & 1], tiles[it & 1], rads[it & 1], lut_k, gtid);
    else decode_v<D, VBITS>(graw[it & 1], tiles[it & 1], rads[it & 1], lut_v, gtid);
  };
  // this group's raw tile it into graw[it & 1] (group 0: K, and with QJL the
  // signs into raw_s[it % 3], one wave instruction)
  auto dma = [&](int it) {
    int rel;
    if (group == 0) {
      dma_raw<VBK>(tile_rsrc(a.k_pages, kres, it * kPT, VBK, rel), graw[it & 1], rel, gw, lane);
      if constexpr (QJL) {
        const __amdgpu_buffer_rsrc_t sr = tile_rsrc(a.s_pages, sres, it * kPT, SGB, rel);
        if (gw == 0 && 16 * lane < kPT * SGB)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (__attribute__((address_space(3))) void *)raw_s[it % 3], 16,
                                                   rel * SGB + 16 * lane, 0, 0, 0);
      }
    } else {
      dma_raw<VBV>(tile_rsrc(a.v_pages, vres, it * kPT, VBV, rel), graw[it & 1], rel, gw, lane);
    }
  };
  auto wait_dma = [] { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); };
  // Block barrier for LDS hand-offs only: __syncthreads' release fence would
  // also wait for the raw-tile copies still in flight.
  auto barrier = [] { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };
  if (ntiles > 0) dma(0);
  if (ntiles > 1) dma(1);
  wait_dma();
  __syncthreads();  // tables and the first two raw tiles ready
  if (ntiles > 0) decode(0);
  __syncthreads();  // tile 0 decoded

  // One loop per group (the compiler then sees that the scores and the
  // weights are never live together); both make 2 ntiles + 2 barrier calls.
  // Raw tile it + 2 streams into LDS from Y(it) on (after tile it + 1's
  // decode freed nothing it needs: it overwrites tile it's raw buffer); each
  // wave waits for its copies before the barrier that ends its next X stage.
  auto x_stage = [&](int it) {
    __builtin_amdgcn_s_setprio(1);
    if (it >= 1) values(it - 1);
    __builtin_amdgcn_sched_barrier(0);  // weights die before the scores start
    if (it < ntiles) scores(it);
    __builtin_amdgcn_s_setprio(0);
    wait_dma();
  };
  auto y_stage = [&](int it) {
    softmax(it);
    if (it + 1 < ntiles) {
      decode(it + 1);
      if (it + 2 < ntiles) dma(it + 2);
    }
  };
  if (ntiles > 0) {
    if (group == 0) {
      for (int it = 0; it <= ntiles; ++it) {
        x_stage(it);                                   // stage 2 it
        barrier();
        if (it < ntiles) y_stage(it);                  // stage 2 it + 1
        barrier();
      }
    } else {
      barrier();                                 // stage 0
      for (int it = 0; it <= ntiles; ++it) {
        x_stage(it);                                   // stage 2 it + 1
        barrier();
        if (it < ntiles) {                             // stage 2 it + 2
          y_stage(it);
          barrier();
        }
      }
    }
  }

  // ---------------- normalise and write o_rot ----------------
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const float l = rows_sum(l_run[rt]);
    float f[4];
    per_row(l > 0.0f ? 1.0f / (l * kPlaneScale) : 0.0f, grp, f);   // the value planes' 2^6 as well
    // output rows 4 grp + i of this row tile
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * RT * wave + 16 * rt + 4 * grp + i;
      const int tok = q0 + row / G, head = row % G;
      if (row < a.qt * G && tok < a.Sq) {
        float *dst = a.o + (((int64_t)(b * a.Hq + h * G + head) * a.Sq) + tok) * D;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) dst[16 * nb + col] = oacc[rt][nb][i] * f[i];
      }
    }
  }
}

template <int D, int KB, int VBITS>
static void launch_pw(const PrefillArgs &a, dim3 grid, hipStream_t s) {
  if (a.qjl != nullptr || a.s_pages != nullptr) prefill_mfma_kernel<D, KB, VBITS, true><<<grid, kPW * 64, 0, s>>>(a);
  else prefill_mfma_kernel<D, KB, VBITS, false><<<grid, kPW * 64, 0, s>>>(a);
}

template <int D>
static void launch_pd(const PrefillArgs &a, int kb, int vb, dim3 grid, hipStream_t s) {
  if (kb == 4 && vb == 4) launch_pw<D, 4, 4>(a, grid, s);
  else if (kb == 4) launch_pw<D, 4, 2>(a, grid, s);
  else if (vb == 4) launch_pw<D, 2, 4>(a, grid, s);
  else launch_pw<D, 2, 2>(a, grid, s);
}

hipError_t launch_prefill(const PrefillArgs &a, int k_bits, int v_bits, hipStream_t s) {
  const int qtiles = (a.Sq + a.qt - 1) / a.qt;
  dim3 grid(qtiles, a.B * a.n_heads);
  if (a.d == 128) launch_pd<128>(a, k_bits, v_bits, grid, s);
  else launch_pd<64>(a, k_bits, v_bits, grid, s);
  return hipGetLastError();
}

int prefill_rows_per_block(bool qjl) { return kPW * (qjl ? kPRowsWave / 2 : kPRowsWave); }

}  // namespace pqkv
