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
// rows 4(l/16)+i, column l%16.
//   scores  S[row][token]: B column = token, a lane's 8 k values = 4
//           coordinates x (hi, lo) = two packed bytes, each read from a
//           256-entry table of (c_hi, c_lo, c_hi', c_lo') for its two codes.
//   values  O[row][coord]: B column = coordinate, a lane's 8 k values = 4
//           tokens x (hi, lo); two tokens' nibbles of that coordinate are
//           interleaved into one byte, so the same kind of table read gives
//           both tokens' (hi, lo) values.
#include "pqkv_device.h"
#include "pqkv_launch.h"

namespace pqkv {

namespace {

constexpr int kMWaves = 4;
constexpr int kChunk = 32;          // tokens per wave iteration
constexpr float kLoScale = 2048.0f; // 2^11

__device__ __forceinline__ void split_hi_lo(float x, half_t *hi, half_t *lo) {
  const half_t h = (half_t)x;
  *hi = h;
  *lo = (half_t)__builtin_fmaf(x, kLoScale, -(float)h * kLoScale);
}

// byte b -> halfs (c_hi[b & 15], c_lo[b & 15], c_hi[b >> 4], c_lo[b >> 4])
__device__ __forceinline__ void build_lut_pairs(uint2 *lut, const float *cb, int tid) {
  if (tid < 256) {
    half_t h0, l0, h1, l1;
    split_hi_lo(cb[tid & 15], &h0, &l0);
    split_hi_lo(cb[tid >> 4], &h1, &l1);
    half2_t a = {h0, l0}, c = {h1, l1};
    lut[tid] = make_uint2(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, c));
  }
}

__device__ __forceinline__ half8_t pack8(uint2 a, uint2 b) {
  typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
  u32x4v v = {a.x, a.y, b.x, b.y};
  return __builtin_bit_cast(half8_t, v);
}

__device__ __forceinline__ float4_t mfma16(half8_t a, half8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Raw buffer over one (batch, head) stream: loads past `bytes` return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t stream_rsrc(const uint8_t *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint32_t bld32(__amdgpu_buffer_rsrc_t r, int off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t bld16(__amdgpu_buffer_rsrc_t r, int off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}

// Raw bytes of one 32-token chunk as this lane needs them.
template <int D>
struct ChunkRegs {
  uint32_t k[2][D / 16];   // per 16-token sub-tile: the two code bytes of MFMA step kk
  uint32_t rk[2], rv[2];   // fp16 radius bits of the lane's score-side tokens
  uint32_t v[8][2];        // value qs dword vw of tokens 4*grp + e (+16 for e >= 4), aligned pair
};

template <int D>
__device__ __forceinline__ void load_chunk(ChunkRegs<D> &c, __amdgpu_buffer_rsrc_t kr, __amdgpu_buffer_rsrc_t vr,
                                           int t0, int col, int grp, int vob_al) {
  constexpr int VB = vector_bytes(D, 4);
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    const int base = (t0 + 16 * st + col) * VB;
    c.rk[st] = bld16(kr, base);
    c.rv[st] = bld16(vr, base);
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk)  // qs bytes 8kk + 2grp, +1
      c.k[st][kk] = bld16(kr, base + (kk >> 1) * kPq4BlockBytes + 2 + 8 * (kk & 1) + 2 * grp);
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int off = (t0 + 16 * (e >> 2) + 4 * grp + (e & 3)) * VB + vob_al;
    c.v[e][0] = bld32(vr, off);
    c.v[e][1] = bld32(vr, off + 4);
  }
}

}  // namespace

template <int D, int G>
__device__ __forceinline__ void process_chunk(const ChunkRegs<D> &cur, int t0, int t_end, int col, int grp, int wave,
                                              int vsh, int vpar, const uint2 *lut_k, const uint2 *lut_v,
                                              half_t (*p_lds)[kChunk][2], const half8_t *qa, float (&m_run)[4],
                                              float (&l_run)[4], float4_t *oacc) {
  constexpr int KK = D / 16;     // score MFMAs per 16-token sub-tile
  constexpr int NB = D / 16;     // value n-tiles
  const int shead0 = 4 * (grp & 1);
  const int ntok = min(kChunk, t_end - t0);

  // ---------------- scores ----------------
  float4_t sacc[2];
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    sacc[st] = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const uint32_t u = cur.k[st][kk];
      sacc[st] = mfma16(qa[kk], pack8(lut_k[u & 0xFF], lut_k[(u >> 8) & 0xFF]), sacc[st]);
    }
  }

  // ---------------- online softmax (rows 0-7 = heads) ----------------
  float s[2][4];
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    const float rk = half_bits_to_float(cur.rk[st]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float cross = shfl_xor_f(sacc[st][i], 32);
      const bool ok = (16 * st + col) < ntok && grp < 2 && (shead0 + i) < G;
      s[st][i] = ok ? __builtin_fmaf(cross, 1.0f / kLoScale, sacc[st][i]) * rk : -INFINITY;
    }
  }
  float alpha[4];
  bool moved = false;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float mx = fmaxf(s[0][i], s[1][i]);
#pragma unroll
    for (int sft = 1; sft < 16; sft <<= 1) mx = fmaxf(mx, shfl_xor_f(mx, sft));
    const float mnew = fmaxf(m_run[i], mx);
    // a head with no valid score yet keeps m = -inf; avoid inf - inf
    alpha[i] = mnew == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run[i] - mnew);
    moved |= mnew != m_run[i];
    float psum = 0.0f;
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const float p = s[st][i] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s[st][i] - mnew);
      psum += p;
      const int head = shead0 + i;
      if (grp < 2 && head < G) {
        half_t ph, pl;
        split_hi_lo(p * half_bits_to_float(cur.rv[st]), &ph, &pl);
        const half2_t top = {ph, (half_t)0.0f}, bot = {pl, ph};
        *(half2_t *)&p_lds[head][16 * st + col][0] = top;
        *(half2_t *)&p_lds[8 + head][16 * st + col][0] = bot;
      }
    }
    l_run[i] = l_run[i] * alpha[i] + psum;
    m_run[i] = mnew;
  }
  // O rows 4*grp + i belong to head 4*(grp & 1) + i: lanes 32-63 take the
  // factors of lanes 0-31. Skipped when no running max moved.
  if (__ballot(moved) != 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float other = shfl_xor_f(alpha[i], 32);
      const float f = grp < 2 ? alpha[i] : other;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) oacc[nb][i] *= f;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // ---------------- values: two 16-token k-blocks ----------------
#pragma unroll
  for (int kb2 = 0; kb2 < 2; ++kb2) {
    const half8_t pa = *(const half8_t *)&p_lds[col][16 * kb2 + 4 * grp][0];
    const uint32_t w0 = align_bytes(cur.v[4 * kb2 + 0][1], cur.v[4 * kb2 + 0][0], vsh);
    const uint32_t w1 = align_bytes(cur.v[4 * kb2 + 1][1], cur.v[4 * kb2 + 1][0], vsh);
    const uint32_t w2 = align_bytes(cur.v[4 * kb2 + 2][1], cur.v[4 * kb2 + 2][0], vsh);
    const uint32_t w3 = align_bytes(cur.v[4 * kb2 + 3][1], cur.v[4 * kb2 + 3][0], vsh);
    // token pairs (0,1), (2,3): byte k of x = even coordinate 2k, of y = odd 2k+1
    const uint32_t x01 = (w0 & 0x0F0F0F0Fu) | ((w1 << 4) & 0xF0F0F0F0u);
    const uint32_t y01 = ((w0 >> 4) & 0x0F0F0F0Fu) | (w1 & 0xF0F0F0F0u);
    const uint32_t x23 = (w2 & 0x0F0F0F0Fu) | ((w3 << 4) & 0xF0F0F0F0u);
    const uint32_t y23 = ((w2 >> 4) & 0x0F0F0F0Fu) | (w3 & 0xF0F0F0F0u);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      // D = 128: n-tile nb is nibble nb of dword col (coordinate 8*col + nb).
      // D = 64: n-tile nb is coordinate 8*(col & 7) + 2*nb + (col >> 3).
      const int par = D == 128 ? (nb & 1) : vpar;
      const int byte = D == 128 ? (nb >> 1) : nb;
      const uint32_t i01 = ((par ? y01 : x01) >> (8 * byte)) & 0xFF;
      const uint32_t i23 = ((par ? y23 : x23) >> (8 * byte)) & 0xFF;
      oacc[nb] = mfma16(pa, pack8(lut_v[i01], lut_v[i23]), oacc[nb]);
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int D, int G>
__global__ void __launch_bounds__(256, 2) decode_mfma_kernel(const DecodeArgs a) {
  constexpr int KK = D / 16;
  constexpr int NB = D / 16;

  __shared__ uint2 lut_k[256], lut_v[256];
  // per wave: P as (hi, 0) in rows 0-7 and (lo, hi) in rows 8-15, per token
  __shared__ __attribute__((aligned(16))) half_t p_lds[kMWaves][16][kChunk][2];
  __shared__ float red_m[kMWaves][8], red_l[kMWaves][8];
  __shared__ float red_o[kMWaves][8][D];

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
  const uint32_t valid_bytes = (uint32_t)a.S * (uint32_t)vector_bytes(D, 4);
  const __amdgpu_buffer_rsrc_t kres = stream_rsrc(kstream, valid_bytes);
  const __amdgpu_buffer_rsrc_t vres = stream_rsrc(vstream, valid_bytes);

  build_lut_pairs(lut_k, a.k_cb + h * a.cb_head_stride, tid);
  build_lut_pairs(lut_v, a.v_cb + h * a.cb_head_stride, tid);
  for (int i = tid; i < kMWaves * 16 * kChunk * 2; i += 256) (&p_lds[0][0][0][0])[i] = (half_t)0.0f;

  // Query fragments: row col = (head col & 7, part col >> 3); k = 8grp + i is
  // (coordinate 16kk + 4grp + i/2, part i%2).
  const int ahead = col & 7;
  const bool arow_lo = col >= 8;
  const float qmask = ahead < G ? 1.0f : 0.0f;
  half8_t qa[KK];
  const float *qrow = a.q + (int64_t)(b * a.Hq + h * G + (ahead < G ? ahead : 0)) * D;
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      half_t vh, vl;
      split_hi_lo(qrow[16 * kk + 4 * grp + j] * qmask, &vh, &vl);
      qa[kk][2 * j] = arow_lo ? vl : vh;
      qa[kk][2 * j + 1] = arow_lo ? vh : (half_t)0.0f;
    }
  }

  float m_run[4], l_run[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m_run[i] = -INFINITY;
    l_run[i] = 0.0f;
  }
  float4_t oacc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) oacc[nb] = (float4_t){0.f, 0.f, 0.f, 0.f};

  // Value-side lane roles: qs dword vw of a lane's tokens.
  const int vw = D == 128 ? col : (col & 7);
  const int vpar = D == 128 ? 0 : (col >> 3);   // D = 64: even / odd coordinates
  const int vob = (vw >> 2) * kPq4BlockBytes + 2 + 4 * (vw & 3);
  const int vob_al = vob & ~3, vsh = vob & 3;
  __syncthreads();

  // Two register sets alternate: one is consumed while the next chunk of
  // this wave streams into the other.
  ChunkRegs<D> ra, rb;
  constexpr int kStep = kMWaves * kChunk;
  int t0 = t_begin + wave * kChunk;
  if (t0 < t_end) load_chunk<D>(ra, kres, vres, t0, col, grp, vob_al);
  while (t0 < t_end) {
    if (t0 + kStep < t_end) load_chunk<D>(rb, kres, vres, t0 + kStep, col, grp, vob_al);
    process_chunk<D, G>(ra, t0, t_end, col, grp, wave, vsh, vpar, lut_k, lut_v, p_lds[wave], qa, m_run, l_run,
                        oacc);
    t0 += kStep;
    if (t0 >= t_end) break;
    if (t0 + kStep < t_end) load_chunk<D>(ra, kres, vres, t0 + kStep, col, grp, vob_al);
    process_chunk<D, G>(rb, t0, t_end, col, grp, wave, vsh, vpar, lut_k, lut_v, p_lds[wave], qa, m_run, l_run,
                        oacc);
    t0 += kStep;
  }

  // ---------------- per-wave results ----------------
  const int shead0 = 4 * (grp & 1);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float l = l_run[i];
#pragma unroll
    for (int sft = 1; sft < 16; sft <<= 1) l += shfl_xor_f(l, sft);
    l_run[i] = l;
  }
  if (grp < 2 && col == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (shead0 + i < G) {
        red_m[wave][shead0 + i] = m_run[i];
        red_l[wave][shead0 + i] = l_run[i];
      }
    }
  }
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float cross = shfl_xor_f(oacc[nb][i], 32);
      const int head = shead0 + i;
      if (grp < 2 && head < G) {
        const int coord = D == 128 ? 8 * col + nb : 8 * (col & 7) + 2 * nb + (col >> 3);
        red_o[wave][head][coord] = __builtin_fmaf(cross, 1.0f / kLoScale, oacc[nb][i]);
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
      O += red_o[w][hh][c] * sc;
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
