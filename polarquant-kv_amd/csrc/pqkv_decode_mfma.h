// Split-K decode attention on the matrix cores (gfx950 v_mfma_f32_16x16x32_f16)
// (kernel templates; the instantiations are spread over the
// pqkv_decode_mfma*.hip translation units so that they compile in parallel)
// for block_pq4 / block_pq2 keys and values, optionally with the QJL sign
// correction on the keys.
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
// 2-bit codes: a nibble holds two codes, so the same operand shapes come from
// 16-entry tables (nibble -> (c_hi, c_lo, c_hi', c_lo')); value tokens pair
// up as two crumbs per nibble.
// QJL: s += [e != 0] sum_i (2 sign_i - 1) pq_i with pq = P_rot q / m, a
// second product on the matrix cores: A = the signs as +-1 (a 16-entry table
// maps 4 sign bits to 4 halves), B = pq as (hi | lo) columns, 32 projections
// per MFMA. A zero residual e projects to P 0 = 0 >= 0, all m signs 1; the
// block cache keeps no residual norm, so an all-ones sketch is read as e = 0
// and gets no correction (the reference's guard, python/polarquant_kv/
// qjl.py:50-51): one ballot per sub-tile, its four lane-group slices ANDed.
// Operands come straight from HBM in MFMA lane order (no LDS staging): a key
// lane loads its lane group's qs bytes of one token (lane group grp owns
// coordinates grp*D/4 .. grp*D/4 + D/4 - 1, so they are contiguous), a value
// lane its qs word of four tokens, and each lane one radius that DPP row
// broadcasts hand to the lanes of its score rows. LDS holds only the code
// tables, each entry stored once per lane of a half-wave (bank-sliced) so
// that random lookups are conflict-free. Cross-lane steps use DPP row rotations / broadcasts and the gfx950
// permlane16/32 swaps (VALU); ds_bpermute moves the rare rescale factors.
// With G <= 4 a score row has only four live head lanes, so the softmax of a
// chunk runs on the four sub-tiles' logits compacted into one register set
// (bank-masked DPP row shifts) and is spread back per sub-tile.
#pragma once

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

// 4-bit: byte b -> halfs (c_hi[b & 15], c_lo[b & 15], c_hi[b >> 4], c_lo[b >> 4]);
// 2-bit: nibble n -> the same for codes n & 3 and n >> 2.
// `levels` < 2^BITS: a codebook of that many entries (codes past it read 0).
template <int BITS>
__device__ __forceinline__ void build_lut_pairs(uint2 *lut, const float *cb, int tid, int levels = 1 << BITS) {
  constexpr int N = BITS == 4 ? 256 : 16, SH = BITS == 4 ? 4 : 2, MASK = BITS == 4 ? 15 : 3;
  auto c = [&](int i) { return levels >= (1 << BITS) || i < levels ? cb[i] : 0.0f; };
  if (tid < N) {
    half_t h0, l0, h1, l1;
    split_hi_lo(c(tid & MASK), &h0, &l0);
    split_hi_lo(c(tid >> SH), &h1, &l1);
    lut[tid] = make_uint2(pack_h2(h0, l0), pack_h2(h1, l1));
  }
}

// Bank-sliced tables. A lookup of random 8-byte entries by 64 lanes runs
// into bank conflicts (~4.4 clk per wave read against ~2.7 conflict-free on
// gfx950, measured under full load). Storing each entry 32 times, copy c at
// uint2 index 32 e + c, gives the 32 lanes of a half-wave (copy lane & 31)
// 32 different bank pairs. A lane's byte address for entry e is
// e * 256 + (lane & 31) * 8, one byte permute from a code byte (slice_addr).
constexpr int kSlices = 32;

// 4-bit pairs, 8192 slots: thread t (< 256) writes slots t + 256 j, j < 32,
// which hold entry e = (t >> 5) + 8 j: e & 15 = (t >> 5) + 8 (j & 1) and
// e >> 4 = j >> 1 (the codebook reads of the j loop are uniform).
// `levels` < 16: a codebook of that many entries (codes past it read 0).
__device__ __forceinline__ void build_sliced4(uint2 *tab, const float *cb, int tid, int levels = 16) {
  auto c = [&](int i) { return levels >= 16 || i < levels ? cb[i] : 0.0f; };
  const int r = tid >> 5;
  half_t h, l;
  split_hi_lo(c(r), &h, &l);
  const uint32_t pa = pack_h2(h, l);
  split_hi_lo(c(r + 8), &h, &l);
  const uint32_t pb = pack_h2(h, l);
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    split_hi_lo(c(j >> 1), &h, &l);
    tab[tid + 256 * j] = make_uint2((j & 1) ? pb : pa, pack_h2(h, l));
  }
}

// 2-bit pairs, 512 slots: nibble e -> codes e & 3 and e >> 2.
__device__ __forceinline__ void build_sliced2(uint2 *tab, const float *cb, int tid) {
#pragma unroll
  for (int i = tid; i < 16 * kSlices; i += 256) {
    const int e = i >> 5;
    half_t h0, l0, h1, l1;
    split_hi_lo(cb[e & 3], &h0, &l0);
    split_hi_lo(cb[e >> 2], &h1, &l1);
    tab[i] = make_uint2(pack_h2(h0, l0), pack_h2(h1, l1));
  }
}

// QJL, 512 slots: 4 sign bits e -> the halfs (2 bit_j - 1), j = 0..3.
__device__ __forceinline__ void build_sliced_sign(uint2 *tab, int tid) {
#pragma unroll
  for (int i = tid; i < 16 * kSlices; i += 256) {
    const int e = i >> 5;
    uint32_t h[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) h[j] = ((e >> j) & 1) ? 0x3C00u : 0xBC00u;  // +1.0 / -1.0 fp16
    tab[i] = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
  }
}

// Byte address in a sliced table of the entry indexed by byte k of w:
// (byte k) << 8 | loff, loff = (lane & 31) * 8.
__device__ __forceinline__ uint32_t slice_addr(uint32_t w, uint32_t loff, int k) {
  return __builtin_amdgcn_perm(w, loff, 0x0C0C0000u | ((4u + (uint32_t)k) << 8));
}
__device__ __forceinline__ uint2 slice_read(const uint2 *tab, uint32_t addr) {
  return *(const uint2 *)((const char *)tab + addr);
}
// Nibble indices as bytes: byte k of the result is nibble 2k (lo) or 2k + 1.
__device__ __forceinline__ uint32_t nib_lo(uint32_t w) { return w & 0x0F0F0F0Fu; }
__device__ __forceinline__ uint32_t nib_hi(uint32_t w) { return (w >> 4) & 0x0F0F0F0Fu; }

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
// Every lane has a source, so no "old" value is needed (mov_dpp with
// bound_ctrl: no zero-initialised copy, and the move can fold into its user).
__device__ __forceinline__ uint32_t row_ror8(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x128, 0xF, 0xF, true);
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
__device__ __forceinline__ uint32_t bld32(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ uint32_t bld16(__amdgpu_buffer_rsrc_t r, int off) {
  return (uint32_t)__builtin_bit_cast(uint16_t, __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0));
}

// N consecutive dwords at byte offset `off`, which need only be 2-byte
// aligned: buffer loads at 2 mod 4 return the bytes at that address (checked
// on gfx950), so the qs words of a block need no realignment.
template <int N>
__device__ __forceinline__ void load_words(__amdgpu_buffer_rsrc_t r, int off, uint32_t (&w)[N]) {
  typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
  if constexpr (N == 4) {
    const u32x4 x = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
    w[0] = x.x; w[1] = x.y; w[2] = x.z; w[3] = x.w;
  } else if constexpr (N == 2) {
    const u32x2v x = __builtin_bit_cast(u32x2v, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
    w[0] = x.x; w[1] = x.y;
  } else {
    static_assert(N == 1, "operand word count");
    w[0] = bld32(r, off);
  }
}

// Lane n of each 16-lane row to the whole row (DPP row_newbcast:n); n must
// fold to a constant after unrolling.
template <int N>
__device__ __forceinline__ float row_bcast_c(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x150 + N, 0xF, 0xF, true));
}
__device__ __forceinline__ float row_bcast(float x, int n) {
  switch (n) {
    case 0: return row_bcast_c<0>(x);   case 1: return row_bcast_c<1>(x);
    case 2: return row_bcast_c<2>(x);   case 3: return row_bcast_c<3>(x);
    case 4: return row_bcast_c<4>(x);   case 5: return row_bcast_c<5>(x);
    case 6: return row_bcast_c<6>(x);   case 7: return row_bcast_c<7>(x);
    case 8: return row_bcast_c<8>(x);   case 9: return row_bcast_c<9>(x);
    case 10: return row_bcast_c<10>(x); case 11: return row_bcast_c<11>(x);
    case 12: return row_bcast_c<12>(x); case 13: return row_bcast_c<13>(x);
    case 14: return row_bcast_c<14>(x); default: return row_bcast_c<15>(x);
  }
}

// DPP move of src into the banks (4-lane groups of each 16-lane row) set in
// BANK; the other lanes keep old. Sources outside the row read 0.
template <int CTRL, int BANK>
__device__ __forceinline__ uint32_t dpp_into(uint32_t old, uint32_t src) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)src, CTRL, 0xF, BANK, true);
}
// Every lane written (lanes without a source get 0): no old value to set up.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t src) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)src, CTRL, 0xF, 0xF, true);
}
template <int CTRL, int BANK>
__device__ __forceinline__ float dpp_intof(float old, float src) {
  return __builtin_bit_cast(float, dpp_into<CTRL, BANK>(__builtin_bit_cast(uint32_t, old), __builtin_bit_cast(uint32_t, src)));
}
constexpr int kDppIdentity = 0xE4;  // quad_perm [0, 1, 2, 3]
// Lane n of each 4-lane quad to the whole quad (DPP quad_perm [n, n, n, n]).
__device__ __forceinline__ float quad_bcast(float x, int n) {
  const int v = __builtin_bit_cast(int, x);
  switch (n) {
    case 0: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(v, 0x00, 0xF, 0xF, true));
    case 1: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(v, 0x55, 0xF, 0xF, true));
    case 2: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(v, 0xAA, 0xF, 0xF, true));
    default: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(v, 0xFF, 0xF, 0xF, true));
  }
}

constexpr int kNSub = kChunk / kSub;

// One 64-token chunk of keys in operand order, straight from HBM. For
// sub-tile st, lane (col, grp) holds the qs bytes of coordinates
// grp*D/4 .. grp*D/4 + D/4 - 1 of token 16 st + col (kWords dwords, loaded
// at their own, possibly 2 mod 4, offset). r: the radius of token 16 (col / 4) + 4 grp + col % 4 (row
// broadcasts hand each lane those of its score rows). sg (QJL): sign bytes
// grp*D/32 .. of token 16 st + col. mw (additive-mask mode): MW dwords of
// fp16 mask values, two per dword, of the tokens whose logits the lane
// holds in the softmax.
template <int D, int KB, bool QJL, int MW = 0>
struct ChunkK {
  static constexpr int kWords = D * KB / 128;
  uint32_t w[kNSub][kWords];
  uint32_t r;
  uint32_t sg[QJL ? kNSub : 1];
  uint32_t mw[MW > 0 ? MW : 1];
};
// Values: for sub-tile kb and e = 0..3, the lane's qs word of token
// 16 kb + 4 grp + e (4-bit: a dword; 2-bit: a half dword). r as for keys.
template <int VBITS>
struct ChunkV {
  uint32_t w[kNSub][4];
  uint32_t r;
};

}  // namespace

// VSH: 4-bit keys and values with one codebook (k_cb == v_cb) read one
// sliced table; 4-bit values with their own codebook use a plain 256-entry
// table (two sliced 64 KB tables would not leave room for two workgroups
// per CU).
// LDS of one workgroup: only the code tables and the end-of-split reduction
// (which reuses the tables' memory): the operands come straight from HBM in
// the lane order the MFMAs want.
template <int D, int G, int KB, int VBITS, bool QJL, bool VSH>
struct DecodeSmem {
  static_assert(!VSH || (KB == 4 && VBITS == 4), "a shared table needs 4-bit keys and values");
  static constexpr int NSK = (KB == 4 ? 256 : 16) * kSlices;              // key table slots
  static constexpr int NSV = VSH ? 1 : VBITS == 4 ? 256 : 16 * kSlices;   // own value table
  union {
    struct {
      uint2 k[NSK], v[NSV], s[QJL ? 16 * kSlices : 1];
    } t;
    float red_o[kMWaves][G * D];
  } u;
  float red_m[kMWaves][8], red_l[kMWaves][8];
};

// One workgroup: split `split` of the (batch, listed head) pair bh.
// SOA: 4-bit keys and values in the reference kernels' layout
// (csrc/flash_turboquant.cu:29-32): per token D/2 packed code bytes
// (coordinate 2i low nibble, 2i + 1 high nibble) in one array and an fp32
// radius in another (a.k_rad / a.v_rad, S_max per stream), instead of
// block_pq4 vectors with fp16 radii.
// GG (the ggml flash-attn-ext layout): tokens a.k_tok_stride / a.v_tok_stride
// bytes apart (the heads of a token interleaved), rows b of the batch grouped
// a.rows_per_seq to a key / value sequence (seq = b / rows_per_seq), and an
// optional fp16 additive mask (a.mask, row b % rows_per_seq of sequence seq)
// added to every logit; a row whose tokens are all masked gives zeros.
// HW (heads per wave): bh is this wave's own pair; each wave streams every
// chunk of the split for its head and writes its partial itself (the four
// waves of a workgroup take four kv heads of the same tokens, which share
// cache lines when a token's heads are interleaved). The code tables are
// built from one codebook shared by all heads (cb_head_stride 0).
// PG (paged caches): a stream's positions live in pages of 2^page_shift
// tokens (>= 64, so a 64-token chunk lies in one page) found through the
// page tables a.k_pages / a.v_pages / a.s_pages; each chunk's loads go
// through a buffer over its own page.
// FREE: the steady-state iteration has no scheduling fences between its
// table reads, softmax weights and products (the mixed-width pair kernel and
// the ggml layout, 3.5 % and 2.4 % faster that way; the other kernels are as
// fast or faster with them).
template <int D, int G, int KB, int VBITS, bool QJL, bool VSH, bool SOA = false, bool GG = false, bool HW = false,
          bool PG = false, bool FREE = false>
__device__ __forceinline__ void decode_mfma_body(const DecodeArgs &a, DecodeSmem<D, G, KB, VBITS, QJL, VSH> &sm,
                                                 const int split, const int bh) {
  static_assert(!SOA || (KB == 4 && VBITS == 4 && !QJL), "the SoA layout carries 4-bit codes and no QJL signs");
  static_assert(!GG || (!SOA && !QJL), "the ggml layout has block-encoded keys and values and no QJL signs");
  static_assert(!HW || GG, "one kv head per wave is a mode of the ggml layout (fp16 block radii, no listed heads)");
  static_assert(!PG || (!SOA && !GG), "paged caches hold block-encoded vectors, one token per vector slot");
  constexpr int VBK = SOA ? D / 2 : vector_bytes(D, KB), VBV = SOA ? D / 2 : vector_bytes(D, VBITS);
  constexpr int KK = D / 16;     // score MFMAs per 16-token tile
  constexpr int NB = D / 16;     // value n-tiles
  constexpr int NSUB = kNSub;
  constexpr int KQ = D / 32;     // QJL MFMAs per 16-token tile (m = d projections)
  // G <= 4: the softmax runs on the compact layout (below), where a lane
  // holds 4 consecutive tokens' logits; otherwise 4 per sub-tile.
  constexpr bool kCompact = G <= 4;
  constexpr int MW = GG ? (kCompact ? 2 : 2 * NSUB) : 0;  // mask dwords per lane and chunk
  // Compact, the mask is added after the compaction, one iteration after the
  // chunk's scores, so its words travel with the scores (MC of them);
  // otherwise the score product adds it while the chunk's words are loaded.
  constexpr int MC = GG && kCompact ? MW : 1;
  using CK = ChunkK<D, KB, QJL, MW>;
  using CV = ChunkV<VBITS>;

  const uint2 *lut_k = sm.u.t.k, *lut_v = VSH ? sm.u.t.k : sm.u.t.v, *lut_s = sm.u.t.s;
  auto &red_m = sm.red_m;
  auto &red_l = sm.red_l;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int b = bh / a.n_heads, hi_ = bh - b * a.n_heads;
  const bool listed = !GG && a.listed;  // (the ggml layout lists no heads)
  const int h = listed ? a.heads[hi_] : hi_;
  const int seq = GG ? b / a.rows_per_seq : b;   // the key / value sequence of row b
  const int t_begin = split * a.tokens_per_split;
  const int t_end = min(a.S, t_begin + a.tokens_per_split);
  const uint8_t *kstream, *vstream;
  if (listed) {
    kstream = a.k_cache + b * a.k_batch_stride + a.k_head_off[hi_];
    vstream = a.v_cache + b * a.v_batch_stride + a.v_head_off[hi_];
  } else {
    kstream = a.k_cache + seq * a.k_batch_stride + h * a.k_head_stride;
    vstream = a.v_cache + seq * a.v_batch_stride + h * a.v_head_stride;
  }
  // bytes between consecutive tokens of a stream
  const int kts = GG ? (int)a.k_tok_stride : VBK, vts = GG ? (int)a.v_tok_stride : VBV;
  const __amdgpu_buffer_rsrc_t kres = stream_rsrc(kstream, (uint32_t)a.S * (uint32_t)kts);
  const __amdgpu_buffer_rsrc_t vres = stream_rsrc(vstream, (uint32_t)a.S * (uint32_t)vts);
  // GG: the mask row of row b (no mask: an empty buffer, every load reads 0)
  __amdgpu_buffer_rsrc_t mres = kres;
  if constexpr (GG) {
    const uint16_t *mrow = a.mask ? a.mask + seq * a.mask_seq_stride + (b - seq * a.rows_per_seq) * a.mask_row_stride
                                  : nullptr;
    mres = stream_rsrc((const uint8_t *)mrow, mrow ? (uint32_t)a.S * 2u : 0u);
  }
  // radii: fp16 inside the blocks, or (SOA) fp32 arrays of S_max per stream
  __amdgpu_buffer_rsrc_t krres = kres, vrres = vres;
  if constexpr (SOA) {
    const int64_t ri = (int64_t)(b * a.Hkv + h) * a.S_max;
    krres = stream_rsrc((const uint8_t *)(a.k_rad + ri), (uint32_t)a.S * 4u);
    vrres = stream_rsrc((const uint8_t *)(a.v_rad + ri), (uint32_t)a.S * 4u);
  }
  auto ld_rad_k = [&](__amdgpu_buffer_rsrc_t kr, int tok) { return SOA ? bld32(krres, tok * 4) : bld16(kr, tok * kts); };
  auto ld_rad_v = [&](__amdgpu_buffer_rsrc_t vr, int tok) { return SOA ? bld32(vrres, tok * 4) : bld16(vr, tok * vts); };
  auto rad = [](uint32_t bits) { return SOA ? __builtin_bit_cast(float, bits) : half_bits_to_float(bits); };
  __amdgpu_buffer_rsrc_t sres = kres;
  if constexpr (QJL && !PG)
    sres = stream_rsrc(a.qjl + ((int64_t)(b * a.Hkv + h) * a.S_max) * (D / 8), (uint32_t)a.S * (uint32_t)(D / 8));
  // The buffer that chunk t0 loads through and t0's position in it: the
  // whole stream, or (PG) the chunk's page, over the page's valid tokens (so
  // loads past S still read 0). The page address is wave-uniform (a scalar
  // load).
  const int64_t prow = PG ? (int64_t)(b * a.Hkv + h) * a.max_pages : 0;
  auto chunk_rsrc = [&](const uint8_t *const *pages, int t0, uint32_t vb, __amdgpu_buffer_rsrc_t whole, int &rel) {
    if constexpr (PG) {
      const int pg = t0 >> a.page_shift, p0 = pg << a.page_shift;
      rel = t0 - p0;
      return stream_rsrc(pages[prow + pg], (uint32_t)min(a.S - p0, 1 << a.page_shift) * vb);
    } else {
      rel = t0;
      return whole;
    }
  };

  if constexpr (KB == 4) build_sliced4(sm.u.t.k, a.k_cb + h * a.cb_head_stride, tid, SOA ? a.cb_levels : 16);
  else build_sliced2(sm.u.t.k, a.k_cb + h * a.cb_head_stride, tid);
  if constexpr (VBITS == 2) build_sliced2(sm.u.t.v, a.v_cb + h * a.cb_head_stride, tid);
  else if constexpr (!VSH) build_lut_pairs<4>(sm.u.t.v, a.v_cb + h * a.cb_head_stride, tid, SOA ? a.cb_levels : 16);
  if constexpr (QJL) build_sliced_sign(sm.u.t.s, tid);
  const uint32_t loff = (uint32_t)(lane & (kSlices - 1)) * 8u;  // this lane's table copy

  // q as the B operand of the score product: column col = (head col & 7,
  // part col >> 3); step kk, k = 8grp + i covers coordinate
  // grp*D/4 + 4kk + i/2 (the lane group's coordinate range), part i%2:
  //   col < 8 : (q_hi, 0)        col >= 8 : (q_lo, q_hi)
  const int qh = col & 7;
  const bool qlo = col >= 8;
  const float qmask = qh < G ? 1.0f : 0.0f;
  const int64_t qrow_i = (int64_t)(b * a.Hq + h * a.gq + a.q_off + (qh < G ? qh : 0));
  const float *qrow = a.q + qrow_i * D;
  half8_t qb[KK];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      half_t vh, vl;
      split_hi_lo(qrow[grp * (D / 4) + 4 * kk + j] * qmask, &vh, &vl);
      qb[kk][2 * j] = qlo ? vl : vh;
      qb[kk][2 * j + 1] = qlo ? vh : (half_t)0.0f;
    }
  }
  // QJL: pq = P_rot q / m as the B operand of the sign product: step kq,
  // k = 8grp + i covers projection grp*D/4 + 8 kq + i (sign byte kq of the
  // lane's piece); column col < 8 holds pq_hi of head col, col >= 8 holds
  // pq_lo (x 2^11) of head col - 8.
  half8_t pb[QJL ? KQ : 1];
  if constexpr (QJL) {
    const float *pqrow = a.pq + qrow_i * D;
#pragma unroll
    for (int kq = 0; kq < KQ; ++kq)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        half_t vh, vl;
        split_hi_lo(pqrow[grp * (D / 4) + 8 * kq + i] * qmask, &vh, &vl);
        pb[kq][i] = qlo ? vl : vh;
      }
  }

  // Running softmax state: lanes with col < 8 own head col (replicated over
  // the four rows).
  float m_run = -INFINITY, l_run = 0.0f;
  // SOA (fp32 radii, any size): the value weights p r_v go to the matrix
  // cores as fp16 hi/lo parts, so they are scaled by vscale = 2^-vexp with
  // vexp the smallest exponent that keeps the largest value radius seen
  // below 2^15; the running output is kept in that scale (rescaled when
  // vexp grows) and the scale is undone when the wave writes its result.
  // With fp16 block radii (<= 65504) vexp stays 0.
  int vexp = 0;
  float vscale = 1.0f;
  float4_t oacc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) oacc[nb] = (float4_t){0.f, 0.f, 0.f, 0.f};

  // Key side: the lane group's qs bytes start kphys bytes into the vector
  // (2 mod 4 or 0 mod 4).
  auto kphys_of = [](int g) {
    const int kc0 = g * (D / 4);
    return SOA ? kc0 / 2 : (kc0 / kBlock) * block_bytes(KB) + 2 + (kc0 % kBlock) * KB / 8;
  };
  // GG: a token's kv heads sit side by side, so the four lanes of a quad
  // load the four groups of one token (one or two lines) instead of one group
  // of four tokens (four lines), and a lane permute (kperm) hands each lane
  // its own group before the table reads: the lane of token t, group g
  // loads for lane 16 g + t.
  const int kphys = kphys_of(GG ? (lane & 3) : grp);
  const int ktok = GG ? (lane >> 2) : col;
  const int kperm = (4 * col + grp) * 4;
  // Value side: the lane's 8 coordinates (D = 128: 8 col .. + 7; D = 64:
  // 8 (col & 7) .. + 7 with parity col >> 3) as a qs dword (4-bit) or half
  // dword (2-bit) of each token.
  const int vw = D == 128 ? col : (col & 7);
  const int vpar = D == 128 ? 0 : (col >> 3);
  const int vob = SOA ? 4 * vw
                      : VBITS == 4 ? (vw >> 2) * kPq4BlockBytes + 2 + 4 * (vw & 3)
                                   : (vw >> 2) * kPq2BlockBytes + 2 + 2 * (vw & 3);
  // token (relative to the chunk) whose radii this lane loads
  const int rtok = kSub * (col >> 2) + 4 * grp + (col & 3);

  // Every load is unconditional (tokens past S read zeros); a conditional
  // load makes the compiler keep the register array in scratch.
  // Per sub-tile pieces, so that a step can reload each sub-tile's registers
  // as soon as it has read them (and the radii first: they are converted at
  // the start of a step).
  // (kr / vr / sr: the chunk's buffers, t0 its position in them)
  auto load_k_sub = [&](CK &c, __amdgpu_buffer_rsrc_t kr, __amdgpu_buffer_rsrc_t sr, int t0, int st) {
    load_words(kr, (t0 + kSub * st + ktok) * kts + kphys, c.w[st]);
    if constexpr (QJL) {
      const int so = (t0 + kSub * st + col) * (D / 8) + grp * (D / 32);
      c.sg[st] = D == 128 ? bld32(sr, so) : bld16(sr, so);
    }
  };
  auto load_v_sub = [&](CV &c, __amdgpu_buffer_rsrc_t vr, int t0, int kb) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int off = (t0 + kSub * kb + 4 * grp + e) * vts + vob;
      c.w[kb][e] = VBITS == 4 ? bld32(vr, off) : bld16(vr, off);
    }
  };
  // GG: the mask values of the chunk's logits this lane holds in the
  // softmax: compact, tokens 16 (col / 4) + 4 grp .. + 3; otherwise tokens
  // 16 st + 4 grp .. + 3 of every sub-tile st. One 2-byte load per token,
  // so a token is either wholly inside the row (S values) or reads 0.
  auto load_mask = [&](CK &c, int t0) {
    if constexpr (GG) {
#pragma unroll
      for (int j = 0; j < MW; ++j) {
        const int tok = t0 + kSub * (kCompact ? (col >> 2) : j >> 1) + 4 * grp + 2 * (j & 1);
        c.mw[j] = bld16(mres, 2 * tok) | (bld16(mres, 2 * tok + 2) << 16);
      }
    }
  };
  // fp16 mask value j of a lane's mask words, and the logits' exp2 scale
  constexpr float kLog2eF = 1.4426950408889634f;
  auto mask_val = [](const uint32_t *mk, int j) { return half_bits_to_float(mk[j >> 1] >> (16 * (j & 1))); };
  // the key (and sign) buffers of chunk t0 and its position in them (key
  // and sign pages share the page index)
  auto key_rsrc = [&](int t0, __amdgpu_buffer_rsrc_t &sr, int &rel) {
    if constexpr (QJL && PG) {
      int srel;
      sr = chunk_rsrc(a.s_pages, t0, D / 8, sres, srel);
    } else {
      sr = sres;
    }
    return chunk_rsrc(a.k_pages, t0, VBK, kres, rel);
  };
  auto load_k = [&](CK &c, int t0) {
    int rel;
    __amdgpu_buffer_rsrc_t sr;
    const __amdgpu_buffer_rsrc_t kr = key_rsrc(t0, sr, rel);
    c.r = ld_rad_k(kr, rel + rtok);
    load_mask(c, t0);
#pragma unroll
    for (int st = 0; st < NSUB; ++st) load_k_sub(c, kr, sr, rel, st);
  };
  auto load_v = [&](CV &c, int t0) {
    int rel;
    const __amdgpu_buffer_rsrc_t vr = chunk_rsrc(a.v_pages, t0, VBV, vres, rel);
    c.r = ld_rad_v(vr, rel + rtok);
#pragma unroll
    for (int kb = 0; kb < NSUB; ++kb) load_v_sub(c, vr, rel, kb);
  };
  __syncthreads();

  // ---- building blocks of one chunk ----
  // G <= 4 without QJL: the score products leave the MFMA raw (hi part in
  // lanes col < 4, cross part in lanes 8..11) and fbegin combines them after
  // compacting the four sub-tiles, on 4 values per lane instead of 16.
  constexpr bool kRawScores = G <= 4 && !QJL;
  // Table reads of key sub-tile st: per score step kk, 4 codes x (hi, lo)
  // (two 8-byte entries); QJL adds the sign-table reads.
  struct KTile {
    uint2 t[KK][2];
    uint2 s[QJL ? KQ : 1][2];
    uint32_t zf;   // QJL: bit i set = the lane's score row i has an all-ones sketch
  };
  auto kread = [&](const CK &k, int st, KTile &kt) {
    // the lane group's qs words of token 16st + col
    uint32_t qw[CK::kWords];
#pragma unroll
    for (int i = 0; i < CK::kWords; ++i)
      qw[i] = GG ? (uint32_t)__builtin_amdgcn_ds_bpermute(kperm, (int)k.w[st][i]) : k.w[st][i];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      // step kk: coordinates 4kk .. 4kk + 3 of the lane group's range
      if constexpr (KB == 4) {
        const uint32_t w = qw[kk >> 1];
        const int e = kk & 1;
        kt.t[kk][0] = slice_read(lut_k, slice_addr(w, loff, 2 * e));
        kt.t[kk][1] = slice_read(lut_k, slice_addr(w, loff, 2 * e + 1));
      } else {
        // nibbles 2e and 2e + 1 of word kk / 4
        const uint32_t w = qw[kk >> 2];
        const int e = kk & 3;
        kt.t[kk][0] = slice_read(lut_k, slice_addr(nib_lo(w), loff, e));
        kt.t[kk][1] = slice_read(lut_k, slice_addr(nib_hi(w), loff, e));
      }
    }
    if constexpr (QJL) {
      // token 16 st + col has an all-ones sketch when the four lane groups'
      // sign words of it are all ones: bit col of the ballot's four 16-lane
      // slices ANDed; the lane's score rows are tokens 4 grp .. 4 grp + 3
      const uint32_t full = D == 128 ? 0xFFFFFFFFu : 0xFFFFu;
      const uint64_t bal = __builtin_amdgcn_ballot_w64(k.sg[st] == full);
      const uint32_t ones = (uint32_t)(bal & (bal >> 16) & (bal >> 32) & (bal >> 48)) & 0xFFFFu;
      kt.zf = ones >> (4 * grp);
      // sign byte kq: low nibble, high nibble
      const uint32_t slo = nib_lo(k.sg[st]), shi = nib_hi(k.sg[st]);
#pragma unroll
      for (int kq = 0; kq < KQ; ++kq) {
        kt.s[kq][0] = slice_read(lut_s, slice_addr(slo, loff, kq));
        kt.s[kq][1] = slice_read(lut_s, slice_addr(shi, loff, kq));
      }
    }
  };
  // Score products of key sub-tile st, finished to the exp2-domain logit:
  // s = (D[t][h] + 2^-11 D[t][h + 8]) r_k (+ the QJL term unless e = 0) for
  // token 16st + 4grp + i, meaningful in lanes col < G. Lanes of absent heads
  // (q = 0) and the cross lanes (col >= 8) carry finite values that only
  // reach discarded output rows. rkl: this lane's loaded radius.
  auto kmma = [&](const KTile &kt, float rkl, int st, const uint32_t *mk, float4_t &out) {
    float4_t acc = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) acc = mfma16(pack8(kt.t[kk][0], kt.t[kk][1]), qb[kk], acc);
    float4_t accq = (float4_t){0.f, 0.f, 0.f, 0.f};
    if constexpr (QJL) {
#pragma unroll
      for (int kq = 0; kq < KQ; ++kq) accq = mfma16(pack8(kt.s[kq][0], kt.s[kq][1]), pb[kq], accq);
    }
    if constexpr (kRawScores) {
      out = acc;  // combined after the compaction (fbegin)
      return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float rk = row_bcast(rkl, 4 * st + i);  // radius of token 16st + 4grp + i
      float v = __builtin_fmaf(row_ror8f(acc[i]), 1.0f / kLoScale, acc[i]) * rk;
      if constexpr (QJL) {
        const float q = __builtin_fmaf(row_ror8f(accq[i]), 1.0f / kLoScale, accq[i]);
        v = ((kt.zf >> i) & 1u) ? v : v + q;  // zero residuals get no correction
      }
      if constexpr (GG) v = __builtin_fmaf(mask_val(mk, 4 * st + i), kLog2eF, v);  // additive mask, exp2 domain
      out[i] = v;
    }
  };
  // Table reads of value k-block kb: two tokens' codes of the lane's
  // coordinate interleaved into one byte (4-bit) or nibble (2-bit), token
  // pairs (0,1) and (2,3).
  struct VTile {
    uint2 t[NB][2];
  };
  auto vread = [&](const CV &v, int kb, VTile &vt) {
    uint32_t x01, y01, x23, y23;
    if constexpr (VBITS == 4) {
      const uint32_t (&wv)[4] = v.w[kb];
      // byte k of x = even coordinate 2k of both tokens, of y = odd 2k + 1
      x01 = (wv[0] & 0x0F0F0F0Fu) | ((wv[1] << 4) & 0xF0F0F0F0u);
      y01 = ((wv[0] >> 4) & 0x0F0F0F0Fu) | (wv[1] & 0xF0F0F0F0u);
      x23 = (wv[2] & 0x0F0F0F0Fu) | ((wv[3] << 4) & 0xF0F0F0F0u);
      y23 = ((wv[2] >> 4) & 0x0F0F0F0Fu) | (wv[3] & 0xF0F0F0F0u);
    } else {
      const uint32_t (&wv)[4] = v.w[kb];
      // nibble k of x = even coordinate 2k of both tokens, of y = odd 2k + 1
      x01 = (wv[0] & 0x3333u) | ((wv[1] << 2) & 0xCCCCu);
      y01 = ((wv[0] >> 2) & 0x3333u) | (wv[1] & 0xCCCCu);
      x23 = (wv[2] & 0x3333u) | ((wv[3] << 2) & 0xCCCCu);
      y23 = ((wv[2] >> 2) & 0x3333u) | (wv[3] & 0xCCCCu);
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      // D = 128: n-tile nb is coordinate 8*col + nb of the lane's group.
      // D = 64: n-tile nb is coordinate 8*(col & 7) + 2*nb + (col >> 3).
      const int par = D == 128 ? (nb & 1) : vpar;
      const int sub = D == 128 ? (nb >> 1) : nb;
      if constexpr (VBITS == 4 && VSH) {
        vt.t[nb][0] = slice_read(lut_v, slice_addr(par ? y01 : x01, loff, sub));
        vt.t[nb][1] = slice_read(lut_v, slice_addr(par ? y23 : x23, loff, sub));
      } else if constexpr (VBITS == 4) {
        vt.t[nb][0] = lut_v[((par ? y01 : x01) >> (8 * sub)) & 0xFF];
        vt.t[nb][1] = lut_v[((par ? y23 : x23) >> (8 * sub)) & 0xFF];
      } else {
        // nibble sub: byte sub / 2 of the low (even) or high (odd) nibbles
        const uint32_t w01 = par ? y01 : x01, w23 = par ? y23 : x23;
        vt.t[nb][0] = slice_read(lut_v, slice_addr((sub & 1) ? nib_hi(w01) : nib_lo(w01), loff, sub >> 1));
        vt.t[nb][1] = slice_read(lut_v, slice_addr((sub & 1) ? nib_hi(w23) : nib_lo(w23), loff, sub >> 1));
      }
    }
  };
  // Softmax bookkeeping of one chunk: logits sv (tokens >= ntok masked when
  // partial), the new running max, the rescale of the running output.
  //
  // With G <= 4 only lanes col < 4 of a row carry real logits (heads 0-3),
  // so the four sub-tiles' logits are compacted into one register set: lane
  // 4 j + h of a row holds head h of sub-tile j (three DPP row shifts into
  // single banks per value). The maximum, the weights and their hi / lo
  // split then run on 4 values per lane instead of 16, and each sub-tile's
  // A operand is spread back by two bank-masked DPP moves per value. The
  // running max and sum are kept per lane of the compact layout (head
  // col % 4; the sum is reduced across the banks at the end).
  struct FState {
    float mnew, alpha, psum;
    uint32_t top[kCompact ? 4 : 1], bot[kCompact ? 4 : 1];  // compact weights: (p_hi, 0), (p_lo, p_hi)
  };
  // rks (kRawScores): this lane's loaded key radius of the chunk in sc; mk
  // (GG): its mask words of that chunk.
  auto fbegin = [&](float (&sv)[NSUB][4], const float4_t (&sc)[NSUB], int ntok, bool partial, float rvl, float rks,
                    const uint32_t (&mk)[MC]) {
    FState f;
    float cmax;
    float cv[4];
    if constexpr (kCompact) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float c = sc[0][i];
        c = dpp_intof<0x114, 0x2>(c, sc[1][i]);  // row_shr:4 into bank 1
        c = dpp_intof<0x118, 0x4>(c, sc[2][i]);  // row_shr:8 into bank 2
        c = dpp_intof<0x11C, 0x8>(c, sc[3][i]);  // row_shr:12 into bank 3
        if constexpr (kRawScores) {
          // cross parts (lanes 8 + h of sub-tile j) to lane 4 j + h
          float x = sc[2][i];
          x = dpp_intof<0x108, 0x1>(x, sc[0][i]);  // row_shl:8 into bank 0
          x = dpp_intof<0x104, 0x2>(x, sc[1][i]);  // row_shl:4 into bank 1
          x = dpp_intof<0x114, 0x8>(x, sc[3][i]);  // row_shr:4 into bank 3
          // radius of token 16 j + 4 grp + i: lane 4 j + i of the quad
          c = __builtin_fmaf(x, 1.0f / kLoScale, c) * quad_bcast(rks, i);
        }
        if constexpr (GG) c = __builtin_fmaf(mask_val(mk, i), kLog2eF, c);  // the logits are in the exp2 domain
        cv[i] = partial && kSub * (col >> 2) + 4 * grp + i >= ntok ? -INFINITY : c;
      }
      cmax = fmaxf(fmaxf(cv[0], cv[1]), fmaxf(cv[2], cv[3]));
      cmax = fmaxf(cmax, __builtin_bit_cast(float, (uint32_t)__builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, cmax), 0x124, 0xF, 0xF, true)));
      cmax = fmaxf(cmax, __builtin_bit_cast(float, (uint32_t)__builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, cmax), 0x128, 0xF, 0xF, true)));
    } else {
#pragma unroll
      for (int st = 0; st < NSUB; ++st)
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[st][i] = sc[st][i];
      if (partial) {
#pragma unroll
        for (int st = 0; st < NSUB; ++st)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (kSub * st + 4 * grp + i >= ntok) sv[st][i] = -INFINITY;
      }
      cmax = sv[0][0];
#pragma unroll
      for (int st = 0; st < NSUB; ++st)
#pragma unroll
        for (int i = 0; i < 4; ++i) cmax = fmaxf(cmax, sv[st][i]);
    }
    // token 0 of the chunk is valid, so after the row reduction every lane's
    // max is finite; the first chunk has m_run = -inf and alpha = 0. With a
    // mask (GG) every logit so far can be -inf: the exponentials then take 0
    // as their reference point (all weights 0) and m_run stays -inf.
    cmax = rows_max(cmax);
    const float mtrue = fmaxf(m_run, cmax);
    f.mnew = GG && mtrue == -INFINITY ? 0.0f : mtrue;
    f.alpha = __builtin_amdgcn_exp2f(m_run - f.mnew);
    f.psum = 0.0f;
    if constexpr (SOA) {
      const float rmax = wave_max(rvl);
      if (rmax > 16384.0f && rmax <= 3.4e38f) {
        const int need = (int)((__builtin_bit_cast(uint32_t, rmax) >> 23) & 0xFF) - 127 - 13;  // rmax 2^-need < 2^15
        if (need > vexp) {
          const float shrink = __builtin_ldexpf(1.0f, vexp - need);
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) oacc[nb] *= shrink;
          vexp = need;
          vscale = __builtin_ldexpf(1.0f, -vexp);
        }
      }
    }
    m_run = mtrue;
    if constexpr (kCompact) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = __builtin_amdgcn_exp2f(cv[i] - f.mnew);
        f.psum += p;
        // r_v of token 16 (col / 4) + 4 grp + i: lane 4 (col / 4) + i of the quad
        const float rv = quad_bcast(rvl, i);
        half_t ph, pl;
        split_hi_lo(p * (SOA ? rv * vscale : rv), &ph, &pl);
        f.top[i] = pack_h2(ph, (half_t)0.0f);
        f.bot[i] = pack_h2(pl, ph);
      }
    }
    // rescale the running output: lane (col, grp) holds rows 4grp + i, i.e.
    // head 4(grp & 1) + i (hi part for grp < 2, cross part for grp >= 2);
    // alpha of head hh sits in lane hh. Skipped (wave-uniform) when no head's
    // maximum moved, the common case once the first chunks are in.
    if (__builtin_amdgcn_ballot_w64(f.alpha != 1.0f) & 0xFFull) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // lane gather (a select between two read-lanes becomes a scratch
        // array indexed by the lane group)
        const float fi = __builtin_bit_cast(
            float, __builtin_amdgcn_ds_bpermute(4 * (4 * (grp & 1) + i), __builtin_bit_cast(int, f.alpha)));
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) oacc[nb][i] *= fi;
      }
    }
    return f;
  };
  // Weights p * r_v of k-block kb in the A layout: col < 8 -> (p_hi, 0),
  // col >= 8 -> (p_lo, p_hi) of head col - 8, taken from lane col - 8.
  auto fweights = [&](const float (&svk)[4], float rvl, int kb, FState &f) {
    uint32_t pa[4];
    if constexpr (kCompact) {
      // lanes col < 8 (banks 0, 1): top of lane 4 kb + col; lanes col >= 8
      // (banks 2, 3): bot of lane 4 kb + col - 8
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t x;
        // the top move writes every bank; banks 2, 3 are then replaced
        switch (kb) {
          case 0: x = dpp_into<0x118, 0xC>(f.top[i], f.bot[i]); break;
          case 1: x = dpp_mov<0x104>(f.top[i]); x = dpp_into<0x114, 0xC>(x, f.bot[i]); break;
          case 2: x = dpp_mov<0x108>(f.top[i]); x = dpp_into<kDppIdentity, 0xC>(x, f.bot[i]); break;
          default: x = dpp_mov<0x10C>(f.top[i]); x = dpp_into<0x104, 0xC>(x, f.bot[i]); break;
        }
        pa[i] = x;
      }
      return pack8u(pa[0], pa[1], pa[2], pa[3]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p = __builtin_amdgcn_exp2f(svk[i] - f.mnew);
      f.psum += p;
      half_t ph, pl;
      const float rv = row_bcast(rvl, 4 * kb + i);  // r_v of token 16kb + 4grp + i
      split_hi_lo(p * (SOA ? rv * vscale : rv), &ph, &pl);
      const uint32_t top = pack_h2(ph, (half_t)0.0f);
      const uint32_t bot = row_ror8(pack_h2(pl, ph));
      pa[i] = col < 8 ? top : bot;
    }
    return pack8u(pa[0], pa[1], pa[2], pa[3]);
  };
  auto vmma = [&](half8_t pav, const VTile &vt) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) oacc[nb] = mfma16(pav, pack8(vt.t[nb][0], vt.t[nb][1]), oacc[nb]);
  };

  // Scores of a whole chunk (the first one): reads one sub-tile ahead.
  auto scores = [&](const CK &k, float4_t (&sc)[NSUB], float &rks, uint32_t (&mks)[MC]) {
    const float rkl = rad(k.r);
    rks = rkl;
#pragma unroll
    for (int j = 0; j < MC; ++j) mks[j] = k.mw[j];
    KTile kt[2];
    kread(k, 0, kt[0]);
#pragma unroll
    for (int st = 0; st < NSUB; ++st) {
      if (st + 1 < NSUB) kread(k, st + 1, kt[(st + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
      kmma(kt[st & 1], rkl, st, k.mw, sc[st]);
    }
  };
  // Softmax update and value product of a whole chunk (the last one).
  auto finish = [&](const CV &v, const float4_t (&sc)[NSUB], float rks, const uint32_t (&mks)[MC],
                    int ntok, bool partial) {
    float sv[NSUB][4];
    const float rvl = rad(v.r);
    FState f = fbegin(sv, sc, ntok, partial, rvl, rks, mks);
    VTile vt[2];
    vread(v, 0, vt[0]);
#pragma unroll
    for (int kb = 0; kb < NSUB; ++kb) {
      if (kb + 1 < NSUB) vread(v, kb + 1, vt[(kb + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
      vmma(fweights(sv[kb], rvl, kb, f), vt[kb & 1]);
    }
    l_run = l_run * f.alpha + f.psum;
  };
  // One steady-state iteration: scores of the chunk in k (into sn) and the
  // finish of the chunk in v with logits sc, sub-tile by sub-tile: both
  // tiles' table reads are issued first, the softmax weights are computed
  // while they are in flight, then the two products run.
  // One iteration; k and v are reloaded in place with the chunks at tk and
  // tv. With kPieceLoads the pieces go out as the iteration consumes them
  // (loads complete in order, so the next iteration's first reads wait only
  // for the first loads: config 4 28.3 -> 27.3 us); the QJL kernels with
  // G > 4 would spill with that schedule and reload after the iteration.
  constexpr bool kPieceLoads = !QJL || G <= 4;
  auto step = [&](CK &k, CV &v, const float4_t (&sc)[NSUB], float rks, const uint32_t (&mks)[MC],
                  float4_t (&sn)[NSUB], float &rkn, uint32_t (&mkn)[MC], int tk, int tv) {
    float sv[NSUB][4];
    const float rkl = rad(k.r), rvl = rad(v.r);
    rkn = rkl;
    // the buffers of the chunks this iteration loads
    int tkr = tk, tvr = tv;
    __amdgpu_buffer_rsrc_t kr = kres, vr = vres, sr = sres;
    if constexpr (kPieceLoads) {
      kr = key_rsrc(tk, sr, tkr);
      vr = chunk_rsrc(a.v_pages, tv, VBV, vres, tvr);
    }
#pragma unroll
    for (int j = 0; j < MC; ++j) mkn[j] = k.mw[j];
    FState f = fbegin(sv, sc, kChunk, false, rvl, rks, mks);
#pragma unroll
    for (int j = 0; j < NSUB; ++j) {
      KTile kt;
      VTile vt;
      kread(k, j, kt);
      vread(v, j, vt);
      if constexpr (kPieceLoads) {
        load_k_sub(k, kr, sr, tkr, j);
        load_v_sub(v, vr, tvr, j);
        if (j == 0) {
          // the radii with the first pieces: issued at the start of the
          // iteration they fetch lines that some of the chunk's later code
          // loads miss again in L2 (+2.6 % HBM traffic)
          k.r = ld_rad_k(kr, tkr + rtok);
          v.r = ld_rad_v(vr, tvr + rtok);
          if constexpr (kCompact) load_mask(k, tk);
        }
      }
      if constexpr (!FREE) __builtin_amdgcn_sched_barrier(0);
      const half8_t pav = fweights(sv[j], rvl, j, f);
      if constexpr (!FREE) __builtin_amdgcn_sched_barrier(0);
      kmma(kt, rkl, j, k.mw, sn[j]);
      vmma(pav, vt);
    }
    l_run = l_run * f.alpha + f.psum;
    // the mask words of the next chunk, once this one's score products have
    // read theirs (the compact layout loads them with the radii)
    if constexpr (GG && !kCompact && kPieceLoads) load_mask(k, tk);
    if constexpr (!kPieceLoads) {
      load_k(k, tk);
      load_v(v, tv);
    }
  };

  // The wave's chunks start at first + i * kStep. Iteration i computes the
  // scores of chunk i + 1 and finishes chunk i (softmax + values), sub-tile
  // by sub-tile, so each one's table-read latency hides behind the other's
  // work. The key registers are reloaded with chunk i + 2 and the value
  // registers with chunk i + 1. Only the last chunk can be partial; it is
  // finished after the loop.
  constexpr int kStep = HW ? kChunk : kMWaves * kChunk;
  // (PG: through a scalar register, so that the chunk positions and with
  // them the page addresses are known to be wave-uniform)
  const int first = t_begin + (HW ? 0 : (PG ? __builtin_amdgcn_readfirstlane(wave) : wave) * kChunk);
  const int nch = first < t_end ? (t_end - first + kStep - 1) / kStep : 0;
  if (nch > 0) {
    CK ck;
    CV cv;
    load_k(ck, first);
    load_v(cv, first);
    float4_t sacc[NSUB];
    float rks;
    uint32_t mks[MC];
    scores(ck, sacc, rks, mks);
    // chunk 1 (a repeat of chunk 0 when there is none: an L2 hit)
    load_k(ck, first + min(1, nch - 1) * kStep);
    for (int i = 0; i + 1 < nch; ++i) {
      float4_t snext[NSUB];
      float rkn;
      uint32_t mkn[MC];
      step(ck, cv, sacc, rks, mks, snext, rkn, mkn, first + min(i + 2, nch - 1) * kStep, first + (i + 1) * kStep);
#pragma unroll
      for (int st = 0; st < NSUB; ++st) sacc[st] = snext[st];
      rks = rkn;
#pragma unroll
      for (int j = 0; j < MC; ++j) mks[j] = mkn[j];
    }
    const int tlast = first + (nch - 1) * kStep;
    finish(cv, sacc, rks, mks, min(kChunk, t_end - tlast), true);
  }

  // ---------------- per-wave results ----------------
  // l: sum over the four rows of lane col (and, compact, over the four
  // banks of a row); m is already row-uniform.
  if constexpr (kCompact) {
    l_run += __builtin_bit_cast(float, (uint32_t)__builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, l_run), 0x124, 0xF, 0xF, true));
    l_run += __builtin_bit_cast(float, (uint32_t)__builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, l_run), 0x128, 0xF, 0xF, true));
  }
  l_run = rows_sum(l_run);
  if constexpr (HW) {
    // the wave's partial of its G heads, straight from the registers
    float *dst = a.part + (((int64_t)(b * a.Hq + h * a.gq + a.q_off) * a.split_stride) + a.split_base + split) * (D + 2);
    const int64_t hstep = (int64_t)a.split_stride * (D + 2);
    if (lane < G) {
      dst[lane * hstep] = m_run;
      dst[lane * hstep + 1] = l_run;
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float cross = shfl_xor_f(oacc[nb][i], 32);
        const int head = 4 * grp + i;
        if (grp < 2 && head < G) {
          const int coord = D == 128 ? 8 * col + nb : 8 * (col & 7) + 2 * nb + (col >> 3);
          dst[head * hstep + 2 + coord] = __builtin_fmaf(cross, 1.0f / kLoScale, oacc[nb][i]);
        }
      }
    return;
  }
  if (lane < G) {
    red_m[wave][lane] = m_run;
    red_l[wave][lane] = l_run;
  }
  // O[head][coord] = D[head] + 2^-11 D[head + 8]: rows 8-15 sit 32 lanes up.
  __syncthreads();  // every wave is done with the tables that red_o overlays
  float *red_o = sm.u.red_o[wave];
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
        const float o = __builtin_fmaf(cross, 1.0f / kLoScale, oacc[nb][i]);
        red_o[head * D + coord] = SOA ? __builtin_ldexpf(o, vexp) : o;
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
      O += sm.u.red_o[w][hh * D + c] * sc;
    }
    float *dst =
        a.part + (((int64_t)(b * a.Hq + h * a.gq + a.q_off + hh) * a.split_stride) + a.split_base + split) * (D + 2);
    if (c == 0) {
      dst[0] = mx;
      dst[1] = L;
    }
    dst[2 + c] = O;
  }
}

// HW: workgroup row y takes the pairs 4y .. 4y + 3, one per wave (n_heads a
// multiple of 4, so the four share the batch row).
template <int D, int G, int KB, int VBITS, bool QJL, bool VSH, bool SOA = false, bool GG = false, bool HW = false,
          bool PG = false>
__global__ void __launch_bounds__(256, kMfmaBlocksPerCU) decode_mfma_kernel(const DecodeArgs a) {
  __shared__ DecodeSmem<D, G, KB, VBITS, QJL, VSH> sm;
  // (read through a scalar register: the buffer resources built from the
  // pair must be wave-uniform, or every load becomes a loop over lanes)
  const int bh = HW ? __builtin_amdgcn_readfirstlane((int)blockIdx.y * kMWaves + (int)(threadIdx.x >> 6))
                    : (int)blockIdx.y;
  decode_mfma_body<D, G, KB, VBITS, QJL, VSH, SOA, GG, HW, PG, GG>(a, sm, blockIdx.x, bh);
}

// Mixed widths whose kv heads are either 4-bit keys and values (a4, one
// shared codebook) or 2-bit keys and values (a2): both groups in one grid,
// rows 0 .. B*a4.n_heads - 1 of blockIdx.y for the first. The two bodies
// share one LDS allocation (a workgroup runs one of them), so two
// workgroups still fit per CU; one launch instead of two saves a launch's
// fill and drain.
template <int D, int G, bool QJL>
__global__ void __launch_bounds__(256, kMfmaBlocksPerCU) decode_mfma_pair_kernel(const DecodeArgs a4,
                                                                                 const DecodeArgs a2) {
  using S4 = DecodeSmem<D, G, 4, 4, QJL, true>;
  using S2 = DecodeSmem<D, G, 2, 2, QJL, false>;
  __shared__ __attribute__((aligned(16))) uint8_t raw[sizeof(S4) > sizeof(S2) ? sizeof(S4) : sizeof(S2)];
  const int n4 = a4.B * a4.n_heads;
  if ((int)blockIdx.y < n4)
    decode_mfma_body<D, G, 4, 4, QJL, true, false, false, false, false, true>(a4, *reinterpret_cast<S4 *>(raw),
                                                                              blockIdx.x, blockIdx.y);
  else
    decode_mfma_body<D, G, 2, 2, QJL, false, false, false, false, false, true>(a2, *reinterpret_cast<S2 *>(raw),
                                                                               blockIdx.x, blockIdx.y - n4);
}


// ---- launch helpers (template; each translation unit instantiates its own) ----

#define PQKV_DM_G_SWITCH(KERNEL, ...)                                     \
  switch (G) {                                                            \
    case 1: KERNEL(1, __VA_ARGS__); break;                                \
    case 2: KERNEL(2, __VA_ARGS__); break;                                \
    case 3: KERNEL(3, __VA_ARGS__); break;                                \
    case 4: KERNEL(4, __VA_ARGS__); break;                                \
    case 5: KERNEL(5, __VA_ARGS__); break;                                \
    case 6: KERNEL(6, __VA_ARGS__); break;                                \
    case 7: KERNEL(7, __VA_ARGS__); break;                                \
    default: KERNEL(8, __VA_ARGS__); break;                               \
  }

template <int D, int KB, int VBITS, bool QJL, bool VSH, bool SOA = false, bool GGML = false, bool HW = false,
          bool PG = false>
static void launch_dm(const DecodeArgs &a, int G, hipStream_t s) {
  dim3 grid(a.splits, HW ? a.B * a.n_heads / kMWaves : a.B * a.n_heads);
#define PQKV_DM_ONE(GG, ...) decode_mfma_kernel<D, GG, KB, VBITS, QJL, VSH, SOA, GGML, HW, PG><<<grid, 256, 0, s>>>(a)
  PQKV_DM_G_SWITCH(PQKV_DM_ONE, 0)
#undef PQKV_DM_ONE
}

// One width pair on both head dims, with or without QJL (PG: paged caches,
// whose QJL signs come through a.s_pages).
template <int KB, int VBITS, bool VSH = false, bool PG = false>
static hipError_t launch_dm_widths(const DecodeArgs &a, hipStream_t s) {
  const bool qjl = PG ? a.s_pages != nullptr : a.qjl != nullptr;
  if (a.d == 128) {
    if (qjl) launch_dm<128, KB, VBITS, true, VSH, false, false, false, PG>(a, a.g, s);
    else launch_dm<128, KB, VBITS, false, VSH, false, false, false, PG>(a, a.g, s);
  } else {
    if (qjl) launch_dm<64, KB, VBITS, true, VSH, false, false, false, PG>(a, a.g, s);
    else launch_dm<64, KB, VBITS, false, VSH, false, false, false, PG>(a, a.g, s);
  }
  return hipGetLastError();
}

// Per-width entry points, one translation unit each.
hipError_t launch_dm_k4v4_shared(const DecodeArgs &a, hipStream_t s);  // one codebook, one sliced table
hipError_t launch_dm_k4v4_own(const DecodeArgs &a, hipStream_t s);     // a value codebook of its own
hipError_t launch_dm_k4v2(const DecodeArgs &a, hipStream_t s);
hipError_t launch_dm_k2v4(const DecodeArgs &a, hipStream_t s);
hipError_t launch_dm_k2v2(const DecodeArgs &a, hipStream_t s);
// Paged caches (uniform widths): 4/4 with one shared table or a value
// codebook of its own, and 2/2.
hipError_t launch_dm_paged_k4v4_shared(const DecodeArgs &a, hipStream_t s);
hipError_t launch_dm_paged_k4v4_own(const DecodeArgs &a, hipStream_t s);
hipError_t launch_dm_paged_k2v2(const DecodeArgs &a, hipStream_t s);

}  // namespace pqkv
