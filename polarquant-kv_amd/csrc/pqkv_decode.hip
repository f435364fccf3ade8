// Split-K ("flash-decoding") attention over a block_pq4 / block_pq2 cache.
//
// Semantics follow the reference decode kernels (csrc/flash_turboquant.cu:
// 27-105, integration/polarquant-kv.patch:277-389): scores are dot products
// of the rotated query with codebook[idx] scaled by the key radius, softmax
// over the sequence, output = sum of weights * codebook[vidx] * value radius,
// all in the rotated space, followed by one inverse rotation.
//
// Mapping (one workgroup = 4 waves = one (batch, kv-head, split)):
//   * every packed token is decoded once and used by all G = Hq/Hkv query
//     heads of its group;
//   * a wave streams 64-token tiles of K and V into its own LDS slots;
//   * scores: lane = token, 256-entry byte -> (code, code) half2 table,
//     v_dot2_f32_f16 against the LDS-resident fp16 query pairs;
//   * online softmax per head with wave reductions, exp2 domain (the query is
//     pre-multiplied by scale * log2(e));
//   * values: lane = (token group, qs dword); two tokens' nibbles are
//     interleaved into one byte so a single table read yields
//     (c[token a], c[token b]) for one coordinate and v_dot2_f32_f16 applies
//     both tokens' weights at once, accumulating in fp32;
//   * per-split (max, sum, unnormalised output) go to the workspace and a
//     merge kernel combines splits, normalises and applies x R.
#include "pqkv_device.h"
#include "pqkv_launch.h"

namespace pqkv {

constexpr int kTile = 64;
constexpr int kWaves = 4;

template <int BITS>
__device__ __forceinline__ void build_lut(float *lut, const float *cb, int tid) {
  // byte -> codebook values of the codes it holds, lowest code first:
  // 4-bit: lut[2b .. 2b+1] = c[b & 15], c[b >> 4]
  // 2-bit: lut[4b .. 4b+3] = c[b & 3], c[(b >> 2) & 3], c[(b >> 4) & 3], c[b >> 6]
  if (tid < 256) {
    if (BITS == 4) {
      lut[2 * tid] = cb[tid & 15];
      lut[2 * tid + 1] = cb[tid >> 4];
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) lut[4 * tid + k] = cb[(tid >> (2 * k)) & 3];
    }
  }
}

// Copy nbytes (multiple of 4) from global to a wave-private LDS slot.
__device__ __forceinline__ void load_tile(uint32_t *dst, const uint8_t *src, int nbytes, bool al16, int lane) {
  if (al16) {
    const int nchunk = nbytes >> 4;
    const u32x4 *s4 = (const u32x4 *)src;
    u32x4 *d4 = (u32x4 *)dst;
    for (int c = lane; c < nchunk; c += kWave) d4[c] = __builtin_nontemporal_load(s4 + c);
    const int tail = (nbytes & 15) >> 2;
    if (lane < tail) dst[(nchunk << 2) + lane] = ((const uint32_t *)src)[(nchunk << 2) + lane];
  } else {
    const int nw = nbytes >> 2;
    const uint32_t *s1 = (const uint32_t *)src;
    for (int c = lane; c < nw; c += kWave) dst[c] = s1[c];
  }
}

// fp32 split-K decode. All arithmetic is fp32 FMA: the codebook values and
// the query are kept in fp32, as the 2e-3 absolute output tolerance on
// outlier-channel caches (outputs of magnitude ~1e2) leaves no room for fp16
// rounding of either operand.
template <int D, int G, int KB, int VBITS, bool QJL>
__global__ void __launch_bounds__(256) decode_split_kernel(const DecodeArgs a) {
  constexpr int VBK = vector_bytes(D, KB), VBV = vector_bytes(D, VBITS);
  constexpr int KW = VBK / 4, VW = VBV / 4;                 // dwords per token
  constexpr int NQK = KB == 4 ? D / 8 : D / 16;             // K qs dwords per token
  constexpr int NQV = VBITS == 4 ? D / 8 : D / 16;          // V qs dwords per token
  constexpr int NG = kWave / NQV;                           // V token groups
  constexpr int CPL = VBITS == 4 ? 8 : 16;                  // V coords per lane
  constexpr int KPB = KB == 4 ? 2 : 4, VPB = VBITS == 4 ? 2 : 4;  // codes per byte
  constexpr int TILE_DW = kTile * (KW + VW);
  constexpr int M = D;                                      // QJL projections
  constexpr int GP = (G + 3) & ~3;                          // padded head count

  __shared__ __attribute__((aligned(16))) float lut_k[256 * KPB];
  __shared__ __attribute__((aligned(16))) float lut_v[256 * VPB];
  __shared__ __attribute__((aligned(16))) float q_lds[G][D];
  __shared__ __attribute__((aligned(16))) uint32_t tiles[kWaves * TILE_DW + 4];
  __shared__ __attribute__((aligned(16))) float pr_lds[kWaves][kTile][GP];
  __shared__ float pq_lds[QJL ? G : 1][QJL ? M : 1];
  // QJL partial sums per 4-bit slice of the sign vector: qt[p][v][h] =
  // sum_j (bit j of v ? +1 : -1) pq[h][4p + j], so a key's correction is
  // M/4 table reads instead of M sign multiplies per head.
  __shared__ __attribute__((aligned(16))) float qt[QJL ? M / 4 : 1][16][GP];
  __shared__ float red_m[kWaves][G], red_l[kWaves][G];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int split = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / a.n_heads, hi = bh - b * a.n_heads;
  const int h = a.listed ? a.heads[hi] : hi;
  const int t_begin = split * a.tokens_per_split;
  const int t_end = min(a.S, t_begin + a.tokens_per_split);

  const uint8_t *kstream, *vstream;
  if (a.listed) {
    kstream = a.k_cache + b * a.k_batch_stride + a.k_head_off[hi];
    vstream = a.v_cache + b * a.v_batch_stride + a.v_head_off[hi];
  } else {
    kstream = a.k_cache + b * a.k_batch_stride + h * a.k_head_stride;
    vstream = a.v_cache + b * a.v_batch_stride + h * a.v_head_stride;
  }
  const bool kal = (((uintptr_t)kstream) & 15) == 0, val = (((uintptr_t)vstream) & 15) == 0;

  build_lut<KB>(lut_k, a.k_cb + h * a.cb_head_stride, tid);
  build_lut<VBITS>(lut_v, a.v_cb + h * a.cb_head_stride, tid);
  for (int i = tid; i < G * D; i += 256) {
    const int hh = i / D, p = i - hh * D;
    q_lds[hh][p] = a.q[(int64_t)(b * a.Hq + h * a.gq + a.q_off + hh) * D + p];
  }
  __syncthreads();
  if (QJL) {
    // pq[h][i] = (p_rot[i] . q_h) / m (q already carries scale * log2(e)),
    // computed once per call for every query head
    for (int i = tid; i < G * M; i += 256) {
      const int hh = i / M, r = i - hh * M;
      pq_lds[hh][r] = a.pq[(int64_t)(b * a.Hq + h * a.gq + a.q_off + hh) * M + r];
    }
    __syncthreads();
    for (int i = tid; i < (M / 4) * 16 * GP; i += 256) {
      const int hh = i % GP, v = (i / GP) & 15, pp = i / (16 * GP);
      float acc = 0.0f;
      if (hh < G) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc += ((v >> j) & 1) ? pq_lds[hh][4 * pp + j] : -pq_lds[hh][4 * pp + j];
      }
      qt[pp][v][hh] = acc;
    }
    __syncthreads();
  }

  uint32_t *ktile = tiles + wave * TILE_DW;
  uint32_t *vtile = ktile + kTile * KW;

  float m_run[G], l_run[G], o[G][CPL];
#pragma unroll
  for (int hh = 0; hh < G; ++hh) {
    m_run[hh] = -INFINITY;
    l_run[hh] = 0.0f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) o[hh][c] = 0.0f;
  }

  // V-phase lane roles: qs dword vw of tokens vg, vg + NG, ...
  const int vw = lane % NQV, vg = lane / NQV;
  const int vob = VBITS == 4 ? (vw >> 2) * kPq4BlockBytes + 2 + 4 * (vw & 3)
                             : (vw >> 1) * kPq2BlockBytes + 2 + 4 * (vw & 1);
  const int vodw = vob >> 2, vosh = vob & 3;

  for (int tile = wave;; tile += kWaves) {
    const int t0 = t_begin + tile * kTile;
    if (t0 >= t_end) break;
    const int ntok = min(kTile, t_end - t0);
    // this lane's key signs (QJL), requested before the tile so the load
    // overlaps the score work; lanes past the tile read zeros
    uint32_t sg[QJL ? M / 32 : 1];
    if (QJL) {
      const uint8_t *sb = a.qjl + ((int64_t)(b * a.Hkv + h) * a.S_max + t0) * (M / 8);
      const __amdgpu_buffer_rsrc_t sr =
          __builtin_amdgcn_make_buffer_rsrc((void *)sb, (short)0, ntok * (M / 8), 0x00020000);
#pragma unroll
      for (int wd = 0; wd < M / 32; ++wd)
        sg[wd] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_raw_buffer_load_b32(sr, lane * (M / 8) + 4 * wd, 0, 0));
    }
    load_tile(ktile, kstream + (int64_t)t0 * VBK, ntok * VBK, kal, lane);
    load_tile(vtile, vstream + (int64_t)t0 * VBV, ntok * VBV, val, lane);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- scores: lane = token ----
    const bool valid = lane < ntok;
    const uint32_t *kt = ktile + lane * KW;
    uint32_t W[KW];
#pragma unroll
    for (int i = 0; i < KW; ++i) W[i] = kt[i];
    const float rk = half_bits_to_float(W[0] & 0xFFFFu);
    float s[G];
#pragma unroll
    for (int hh = 0; hh < G; ++hh) s[hh] = 0.0f;
#pragma unroll
    for (int k = 0; k < NQK; ++k) {
      const int ob = KB == 4 ? (k >> 2) * kPq4BlockBytes + 2 + 4 * (k & 3)
                             : (k >> 1) * kPq2BlockBytes + 2 + 4 * (k & 1);
      const uint32_t w = (ob & 3) ? align_bytes(W[(ob >> 2) + 1], W[ob >> 2], 2) : W[ob >> 2];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t byte = (w >> (8 * j)) & 0xFF;
        const int c0 = (4 * k + j) * KPB;  // first coordinate held by this byte
        if (KB == 4) {
          const float2 e = *(const float2 *)&lut_k[2 * byte];
#pragma unroll
          for (int hh = 0; hh < G; ++hh) {
            const float2 qq = *(const float2 *)&q_lds[hh][c0];
            s[hh] = __builtin_fmaf(e.x, qq.x, s[hh]);
            s[hh] = __builtin_fmaf(e.y, qq.y, s[hh]);
          }
        } else {
          const float4 e = *(const float4 *)&lut_k[4 * byte];
#pragma unroll
          for (int hh = 0; hh < G; ++hh) {
            const float4 qq = *(const float4 *)&q_lds[hh][c0];
            s[hh] = __builtin_fmaf(e.x, qq.x, s[hh]);
            s[hh] = __builtin_fmaf(e.y, qq.y, s[hh]);
            s[hh] = __builtin_fmaf(e.z, qq.z, s[hh]);
            s[hh] = __builtin_fmaf(e.w, qq.w, s[hh]);
          }
        }
      }
    }
#pragma unroll
    for (int hh = 0; hh < G; ++hh) s[hh] *= rk;
    if (QJL) {
      // + (1/m) sum_i (2 sign_i - 1) (P q)_i, skipped for a zero residual
      // (an all-ones sketch: P 0 = 0 >= 0 sets every sign).
      bool zero_res = true;
#pragma unroll
      for (int wd = 0; wd < M / 32; ++wd) zero_res = zero_res && sg[wd] == 0xFFFFFFFFu;
      if (valid && !zero_res) {
#pragma unroll
        for (int wd = 0; wd < M / 32; ++wd) {
          const uint32_t bits = sg[wd];
#pragma unroll
          for (int nb = 0; nb < 8; ++nb) {
            const float *e = qt[8 * wd + nb][(bits >> (4 * nb)) & 15];
#pragma unroll
            for (int h4 = 0; h4 < GP; h4 += 4) {
              const float4 v4 = *(const float4 *)(e + h4);
              const float vv[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
              for (int u = 0; u < 4; ++u)
                if (h4 + u < G) s[h4 + u] += vv[u];
            }
          }
        }
      }
    }
    const float rv = half_bits_to_float(vtile[lane * VW] & 0xFFFFu);
    float alpha[G];
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
      const float sv = valid ? s[hh] : -INFINITY;
      const float mnew = fmaxf(m_run[hh], wave_max(sv));
      alpha[hh] = __builtin_amdgcn_exp2f(m_run[hh] - mnew);
      const float p = valid ? __builtin_amdgcn_exp2f(sv - mnew) : 0.0f;
      l_run[hh] = l_run[hh] * alpha[hh] + p;
      m_run[hh] = mnew;
      pr_lds[wave][lane][hh] = valid ? p * rv : 0.0f;
    }
#pragma unroll
    for (int hh = 0; hh < G; ++hh)
#pragma unroll
      for (int c = 0; c < CPL; ++c) o[hh][c] *= alpha[hh];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- values: lane = (token group vg, qs dword vw) ----
#pragma unroll 2
    for (int j = 0; j < kTile / NG; ++j) {
      const int t = vg + NG * j;
      const uint32_t *pt = vtile + t * VW;
      const uint32_t w = align_bytes(pt[vodw + 1], pt[vodw], vosh);
      float pw[GP];
#pragma unroll
      for (int g4 = 0; g4 < GP; g4 += 4) {
        const float4 v4 = *(const float4 *)&pr_lds[wave][t][g4];
        pw[g4] = v4.x; pw[g4 + 1] = v4.y; pw[g4 + 2] = v4.z; pw[g4 + 3] = v4.w;
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t byte = (w >> (8 * k)) & 0xFF;
        if (VBITS == 4) {
          const float2 e = *(const float2 *)&lut_v[2 * byte];
#pragma unroll
          for (int hh = 0; hh < G; ++hh) {
            o[hh][2 * k] = __builtin_fmaf(pw[hh], e.x, o[hh][2 * k]);
            o[hh][2 * k + 1] = __builtin_fmaf(pw[hh], e.y, o[hh][2 * k + 1]);
          }
        } else {
          const float4 e = *(const float4 *)&lut_v[4 * byte];
#pragma unroll
          for (int hh = 0; hh < G; ++hh) {
            o[hh][4 * k] = __builtin_fmaf(pw[hh], e.x, o[hh][4 * k]);
            o[hh][4 * k + 1] = __builtin_fmaf(pw[hh], e.y, o[hh][4 * k + 1]);
            o[hh][4 * k + 2] = __builtin_fmaf(pw[hh], e.z, o[hh][4 * k + 2]);
            o[hh][4 * k + 3] = __builtin_fmaf(pw[hh], e.w, o[hh][4 * k + 3]);
          }
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // ---- combine token groups, then the four waves ----
#pragma unroll
  for (int sft = NQV; sft < kWave; sft <<= 1)
#pragma unroll
    for (int hh = 0; hh < G; ++hh)
#pragma unroll
      for (int c = 0; c < CPL; ++c) o[hh][c] += shfl_xor_f(o[hh][c], sft);
#pragma unroll
  for (int hh = 0; hh < G; ++hh) l_run[hh] = wave_sum(l_run[hh]);

  __syncthreads();
  float *red_o = (float *)tiles;  // [kWaves][G][D]
  if (vg == 0) {
#pragma unroll
    for (int hh = 0; hh < G; ++hh)
#pragma unroll
      for (int c = 0; c < CPL; ++c) red_o[(wave * G + hh) * D + vw * CPL + c] = o[hh][c];
  }
  if (lane == 0) {
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
      red_m[wave][hh] = m_run[hh];
      red_l[wave][hh] = l_run[hh];
    }
  }
  __syncthreads();
  for (int i = tid; i < G * D; i += 256) {
    const int hh = i / D, c = i - hh * D;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mx = fmaxf(mx, red_m[w][hh]);
    float L = 0.0f, O = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float sc = red_m[w][hh] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(red_m[w][hh] - mx);
      L += red_l[w][hh] * sc;
      O += red_o[(w * G + hh) * D + c] * sc;
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

// Combine splits, normalise and rotate back: out = R^T (sum_s w_s o_s / L).
// Workgroup (hg, cg): kMergeHeads query heads x 32 output columns. One wave
// per head computes the split weights; every workgroup of a head group forms
// the full normalised o_rot (cheap, L2-resident partials) and then its 32
// outputs from the matching 32 columns of R, staged as [32][D + 4] (16-byte
// reads; each 16-lane phase of them covers all 64 banks).
// ROT = false (R == nullptr): the normalised o_rot itself is the output.
template <int D, typename TOUT, bool ROT = true>
__global__ void __launch_bounds__(256) decode_merge_kernel(const float *__restrict__ part,
                                                          const float *__restrict__ R,
                                                          TOUT *__restrict__ out, int BHq, int splits) {
  constexpr int NH = kMergeHeads;
  constexpr int NC = 32;           // output columns per workgroup
  constexpr int RP = D + 4;
  constexpr int RU = NC * D / 4 / 256;   // R float4 loads per thread
  constexpr int OU = NH * D / 256;       // (head, coordinate) sums per thread
  constexpr int SB = 16;                 // splits whose o values are loaded at once
  __shared__ __align__(16) float rs[NC * RP];    // rs[jj][k] = R[k][c0 + jj]
  __shared__ __align__(16) float os[NH * D];
  __shared__ float wts[NH][kMaxSplits];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int head0 = blockIdx.x * NH, c0 = blockIdx.y * NC;
  // Every independent global read goes out before the first wait: the R
  // columns, this wave's split maxima and sums (up to 64 splits), and the
  // first SB splits of the thread's o values.
  float4 rv[RU];
  if constexpr (ROT) {
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const int i = tid + 256 * u, k = i / (NC / 4), j4 = i % (NC / 4);
      rv[u] = *(const float4 *)(R + (int64_t)k * D + c0 + 4 * j4);
    }
  }
  const int hq_w = head0 + wave;
  const float *pw = part + (int64_t)min(hq_w, BHq - 1) * splits * (D + 2);
  const float m0 = lane < splits ? pw[(int64_t)lane * (D + 2)] : -INFINITY;
  const float l0 = lane < splits ? pw[(int64_t)lane * (D + 2) + 1] : 0.0f;
  float ov[OU][SB];
#pragma unroll
  for (int u = 0; u < OU; ++u) {
    const int i = tid + 256 * u, hh = i / D, c = i % D;
    const float *p = part + (int64_t)min(head0 + hh, BHq - 1) * splits * (D + 2) + 2 + c;
#pragma unroll
    for (int sp = 0; sp < SB; ++sp) ov[u][sp] = sp < splits ? p[(int64_t)sp * (D + 2)] : 0.0f;
  }
  if constexpr (ROT) {
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const int i = tid + 256 * u, k = i / (NC / 4), j4 = i % (NC / 4);
      rs[(4 * j4 + 0) * RP + k] = rv[u].x;
      rs[(4 * j4 + 1) * RP + k] = rv[u].y;
      rs[(4 * j4 + 2) * RP + k] = rv[u].z;
      rs[(4 * j4 + 3) * RP + k] = rv[u].w;
    }
  }
  if (hq_w < BHq) {
    float mx = m0;
    for (int sp = lane + 64; sp < splits; sp += 64) mx = fmaxf(mx, pw[(int64_t)sp * (D + 2)]);
    mx = wave_max(mx);
    float L = 0.0f;
    for (int sp = lane; sp < splits; sp += 64) {
      const float ms = sp == lane ? m0 : pw[(int64_t)sp * (D + 2)];
      const float ls = sp == lane ? l0 : pw[(int64_t)sp * (D + 2) + 1];
      const float e = ms == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ms - mx);
      wts[wave][sp] = e;
      L = __builtin_fmaf(e, ls, L);
    }
    L = wave_sum(L);
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    for (int sp = lane; sp < splits; sp += 64) wts[wave][sp] *= inv;
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < OU; ++u) {
    const int i = tid + 256 * u, hh = i / D, c = i % D;
    const int hq = head0 + hh;
    float o = 0.0f;
    if (hq < BHq) {
#pragma unroll
      for (int sp = 0; sp < SB; ++sp)
        if (sp < splits) o = __builtin_fmaf(wts[hh][sp], ov[u][sp], o);
      const float *p = part + (int64_t)hq * splits * (D + 2) + 2 + c;
#pragma unroll 8
      for (int sp = SB; sp < splits; ++sp) o = __builtin_fmaf(wts[hh][sp], p[(int64_t)sp * (D + 2)], o);
    }
    os[i] = o;
  }
  __syncthreads();
  if (!ROT && tid < NH * NC) {
    const int hh = tid / NC, jj = tid % NC;
    const int hq = head0 + hh;
    if (hq < BHq) out[(int64_t)hq * D + c0 + jj] = (TOUT)os[hh * D + c0 + jj];
  }
  if (ROT && tid < NH * NC) {
    const int hh = tid / NC, jj = tid % NC;
    const float4 *orow = (const float4 *)(os + hh * D);
    const float4 *rr = (const float4 *)(rs + jj * RP);
    float acc = 0.0f;
#pragma unroll 4
    for (int k4 = 0; k4 < D / 4; ++k4) {
      const float4 a4 = orow[k4], r4 = rr[k4];
      acc = __builtin_fmaf(a4.x, r4.x, acc);
      acc = __builtin_fmaf(a4.y, r4.y, acc);
      acc = __builtin_fmaf(a4.z, r4.z, acc);
      acc = __builtin_fmaf(a4.w, r4.w, acc);
    }
    const int hq = head0 + hh;
    if (hq < BHq) out[(int64_t)hq * D + c0 + jj] = (TOUT)acc;
  }
}

// Streaming-read probe for the measurement hook: every byte of [p, p + n16
// * 16) read once with 16-byte loads in a grid-stride loop, XOR-folded per
// thread; a store that depends on the fold keeps the loads alive.
__global__ void __launch_bounds__(256) stream_read_kernel(const u32x4 *__restrict__ p, int64_t n16,
                                                          uint32_t *__restrict__ sink) {
  u32x4 acc = {0u, 0u, 0u, 0u};
  const int64_t stride = (int64_t)gridDim.x * 256;
  int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const u32x4 a = p[i], b = p[i + stride], c = p[i + 2 * stride], d = p[i + 3 * stride];
    acc ^= a ^ b ^ c ^ d;
  }
  for (; i < n16; i += stride) acc ^= p[i];
  const uint32_t f = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (f == 0x9E3779B9u) sink[blockIdx.x] = f;
}

hipError_t launch_stream_read(const void *p, size_t bytes, uint32_t *sink, int blocks, hipStream_t s) {
  stream_read_kernel<<<blocks, 256, 0, s>>>((const u32x4 *)p, (int64_t)(bytes / 16), sink);
  return hipGetLastError();
}

__global__ void fill_zero_kernel(uint32_t *p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

// ---------------------------------------------------------------------------
template <int D, int G, int KB, int VB>
static void launch_dqg(const DecodeArgs &a, bool qjl, hipStream_t s) {
  dim3 grid(a.splits, a.B * a.n_heads);
  if (qjl) decode_split_kernel<D, G, KB, VB, true><<<grid, 256, 0, s>>>(a);
  else decode_split_kernel<D, G, KB, VB, false><<<grid, 256, 0, s>>>(a);
}

template <int D, int KB, int VB>
static void launch_dq(const DecodeArgs &a, int G, bool qjl, hipStream_t s) {
  switch (G) {
    case 1: launch_dqg<D, 1, KB, VB>(a, qjl, s); break;
    case 2: launch_dqg<D, 2, KB, VB>(a, qjl, s); break;
    case 3: launch_dqg<D, 3, KB, VB>(a, qjl, s); break;
    case 4: launch_dqg<D, 4, KB, VB>(a, qjl, s); break;
    case 5: launch_dqg<D, 5, KB, VB>(a, qjl, s); break;
    case 6: launch_dqg<D, 6, KB, VB>(a, qjl, s); break;
    case 7: launch_dqg<D, 7, KB, VB>(a, qjl, s); break;
    default: launch_dqg<D, 8, KB, VB>(a, qjl, s); break;
  }
}

template <int D>
static void launch_dd(const DecodeArgs &a, int kb, int vb, int G, bool qjl, hipStream_t s) {
  if (kb == 4 && vb == 4) launch_dq<D, 4, 4>(a, G, qjl, s);
  else if (kb == 4) launch_dq<D, 4, 2>(a, G, qjl, s);
  else if (vb == 4) launch_dq<D, 2, 4>(a, G, qjl, s);
  else launch_dq<D, 2, 2>(a, G, qjl, s);
}

hipError_t launch_decode_split(const DecodeArgs &a, int k_bits, int v_bits, hipStream_t s) {
  const int G = a.g;
  const bool qjl = a.qjl != nullptr;
  if (a.d == 128) launch_dd<128>(a, k_bits, v_bits, G, qjl, s);
  else launch_dd<64>(a, k_bits, v_bits, G, qjl, s);
  return hipGetLastError();
}

hipError_t launch_decode_merge(const float *part, const float *R, void *out, int out_dtype, int BHq, int splits,
                               int d, hipStream_t s) {
  if (splits < 1 || splits > kMaxSplits) return hipErrorInvalidValue;
  const dim3 grid((BHq + kMergeHeads - 1) / kMergeHeads, d / 32);
#define PQKV_MERGE(DD, T, ROT) decode_merge_kernel<DD, T, ROT><<<grid, 256, 0, s>>>(part, R, (T *)out, BHq, splits)
  if (R == nullptr) {
    if (d == 128 && out_dtype == 0) PQKV_MERGE(128, float, false);
    else if (d == 128) PQKV_MERGE(128, half_t, false);
    else if (out_dtype == 0) PQKV_MERGE(64, float, false);
    else PQKV_MERGE(64, half_t, false);
  } else {
    if (d == 128 && out_dtype == 0) PQKV_MERGE(128, float, true);
    else if (d == 128) PQKV_MERGE(128, half_t, true);
    else if (out_dtype == 0) PQKV_MERGE(64, float, true);
    else PQKV_MERGE(64, half_t, true);
  }
#undef PQKV_MERGE
  return hipGetLastError();
}

hipError_t launch_fill_zero(void *p, size_t bytes, hipStream_t s) {
  const int64_t n = (int64_t)(bytes / 4);
  if (n > 0) {
    int64_t g = (n + 255) / 256;
    if (g > 4096) g = 4096;
    fill_zero_kernel<<<(int)g, 256, 0, s>>>((uint32_t *)p, n);
  }
  return hipGetLastError();
}

}  // namespace pqkv
