// The reference's GPU group (min / scale) format, CompressedKVCacheGPU
// (src/polarquant_kv_cuda/types.py:7-21), on gfx950: encode, decode, the
// QJL sketch of the key residual, and attention straight on the packed
// codes (the reference decompresses both caches to fp16 and runs dense
// matmuls, src/polarquant_kv_cuda/attention_kernel.py:62-113; its fused
// CUDA kernels read the same fields, csrc/polarquant_full.cu:45-111).
//
// Format, per vector of d coordinates with ng = ceil(d / gs) groups and
// d_pad = ng gs (compress_kernel.py:100-189):
//   y = clamp(x, +-65000) R^T (fp32), r = |y|, u = y / max(r, 1e-30)
//   (0 where r < 1e-30), zero-padded to d_pad; per group lo = min,
//   s = (max - lo) / L (1 for a flat group), L = 2^bits - 1,
//   code = round_half_even(clamp((u - lo) / s, 0, L));
//   stored: radius fp16 (saturated at 65504), lo and s fp16, codes packed
//   4-bit (coordinate 2i low nibble), 2-bit (v0 | v1<<2 | v2<<4 | v3<<6) or
//   one byte per code for the other widths.
//   QJL residual (keys): e = (y - (code s + lo) max(r, 1e-30)) R with the
//   unrounded fp32 lo and s (compress_kernel.py:166-175).
// Decode: x^ = clamp(((code s16 + lo16) r16) R, +-65504) (fp16 output,
// decompress_kernel.py:10-51).
// Attention, in the rotated space: s_t = scale r_t sum_g (s_tg q.c_tg +
// lo_tg sum_{j in g} q_j) (+ the QJL term), o_rot = sum_t w_t r_t (c_t s_t +
// lo_t), o = o_rot R. The fp32 rotation and the fp32 norm are matrix
// products in the reference (torch matmul / norm) whose summation order the
// library picks; here they are FMA chains in coordinate order and the
// correctly rounded fp32 of an fp64 sum of squares.
#include "pqkv_device.h"
#include "pqkv_launch.h"

namespace pqkv {

namespace {

constexpr int kGW = 4;           // vectors (waves) per workgroup: compress / decompress / sketch / query prep
constexpr int kGMax = 256;       // largest d and d_pad handled by the fused attention
constexpr int kGMaxPad = 512;    // d_pad < 2 d
constexpr int kGPer = kGMax / 64;

__device__ __forceinline__ float ld_in(const void *x, int dt, int64_t i) {
  if (dt == PQKV_F16) return (float)((const half_t *)x)[i];
  if (dt == PQKV_BF16) return __builtin_bit_cast(float, (uint32_t)((const uint16_t *)x)[i] << 16);
  return ((const float *)x)[i];
}
// the format's parameters (radius, lo, s, residual norm): fp16 or fp32
__device__ __forceinline__ float ld_par(const void *p, int dt, int64_t i) {
  return dt == PQKV_F16 ? (float)((const half_t *)p)[i] : ((const float *)p)[i];
}
__device__ __forceinline__ void st_par(void *p, int dt, int64_t i, float v) {
  if (dt == PQKV_F16) ((half_t *)p)[i] = (half_t)v;
  else ((float *)p)[i] = v;
}

// a code's value: the code itself, or (codebook mode) its table entry
template <bool CB>
__device__ __forceinline__ float cval(const float *cbl, uint32_t code) {
  if constexpr (CB) return cbl[code & 15];
  else return (float)code;
}

// storage width of a code: 4 and 2 bits pack, every other width takes a byte
__device__ __host__ __forceinline__ int store_bits(int bits) { return bits == 4 ? 4 : bits == 2 ? 2 : 8; }

// code j of a packed row
__device__ __forceinline__ int code_at(const uint8_t *row, int cb, int j) {
  if (cb == 4) return (row[j >> 1] >> ((j & 1) * 4)) & 15;
  if (cb == 2) return (row[j >> 2] >> ((j & 3) * 2)) & 3;
  return row[j];
}

}  // namespace

// ---------------------------------------------------------------------------
// compress: one wave per vector. Rt = R^T ([k][j] = R[j][k]) so that lane j's
// reads of a row of R are coalesced across the wave.
__global__ void __launch_bounds__(kGW * 64)
    group_gpu_compress_kernel(const void *x, int x_dtype, const float *Rt, const float *R, int64_t n, int d, int bits,
                              int gs, void *radius, uint8_t *codes, void *mins, void *scales, int pdt,
                              float *resid) {
  __shared__ float xs[kGW][kGMax];
  __shared__ float us[kGW][kGMaxPad];
  __shared__ float glo[kGW][kGMaxPad], gsc[kGW][kGMaxPad];
  __shared__ uint8_t cq[kGW][kGMaxPad];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int ng = (d + gs - 1) / gs, dpad = ng * gs;
  const int cb = store_bits(bits);
  const int row_bytes = dpad * cb / 8;
  const float L = (float)((1 << bits) - 1);
  for (int64_t v = (int64_t)blockIdx.x * kGW + w; v < n; v += (int64_t)gridDim.x * kGW) {
    for (int k = lane; k < d; k += 64) {
      const float xf = ld_in(x, x_dtype, v * d + k);
      xs[w][k] = xf > 65000.0f ? 65000.0f : xf < -65000.0f ? -65000.0f : xf;   // NaN stays NaN
    }
    __builtin_amdgcn_wave_barrier();
    float y[kGPer];
    double sq = 0.0;
#pragma unroll
    for (int i = 0; i < kGPer; ++i) {
      const int j = lane + 64 * i;
      y[i] = 0.0f;
      if (j < d) {
        float acc = 0.0f;
        for (int k = 0; k < d; ++k) acc = __builtin_fmaf(xs[w][k], Rt[(int64_t)k * d + j], acc);
        y[i] = acc;
        sq += (double)acc * (double)acc;
      }
    }
    for (int s = 32; s > 0; s >>= 1) sq += __shfl_xor(sq, s, 64);
    const float r = (float)__builtin_sqrt(sq);
    const bool zero = r < 1e-30f;
    const float safe = zero ? 1e-30f : r;
#pragma unroll
    for (int i = 0; i < kGPer; ++i) {
      const int j = lane + 64 * i;
      if (j < d) us[w][j] = zero ? 0.0f : __fdiv_rn(y[i], safe);
    }
    for (int j = d + lane; j < dpad; j += 64) us[w][j] = 0.0f;
    __builtin_amdgcn_wave_barrier();
    for (int g = lane; g < ng; g += 64) {
      float lo = us[w][g * gs], hi = lo;
      for (int k = 1; k < gs; ++k) {
        const float u = us[w][g * gs + k];
        lo = fminf(lo, u);
        hi = fmaxf(hi, u);
      }
      const float range = hi - lo;
      const float sc = range > 0.0f ? __fdiv_rn(range, L) : 1.0f;
      glo[w][g] = lo;
      gsc[w][g] = sc;
      st_par(mins, pdt, v * ng + g, lo);
      st_par(scales, pdt, v * ng + g, sc);
    }
    __builtin_amdgcn_wave_barrier();
    for (int j = lane; j < dpad; j += 64) {
      const int g = j / gs;
      float t;
      {
#pragma clang fp contract(off)
        t = __fdiv_rn(us[w][j] - glo[w][g], gsc[w][g]);
      }
      t = t < 0.0f ? 0.0f : t > L ? L : t;   // clamp, then round half to even
      cq[w][j] = (uint8_t)rintf(t);
    }
    __builtin_amdgcn_wave_barrier();
    uint8_t *crow = codes + v * row_bytes;
    for (int i = lane; i < row_bytes; i += 64) {
      uint32_t b;
      if (cb == 4) b = cq[w][2 * i] | (cq[w][2 * i + 1] << 4);
      else if (cb == 2) b = cq[w][4 * i] | (cq[w][4 * i + 1] << 2) | (cq[w][4 * i + 2] << 4) | (cq[w][4 * i + 3] << 6);
      else b = cq[w][i];
      crow[i] = (uint8_t)b;
    }
    if (lane == 0) st_par(radius, pdt, v, r > 65504.0f ? 65504.0f : r);
    if (resid) {
      // rotated-space residual with the unrounded lo / s, then e = er R
      for (int j = lane; j < d; j += 64) {
        const int g = j / gs;
        float hat;
        {
#pragma clang fp contract(off)
          const float dq = (float)cq[w][j] * gsc[w][g] + glo[w][g];
          hat = dq * safe;
        }
        us[w][j] = hat;
      }
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int i = 0; i < kGPer; ++i) {
        const int j = lane + 64 * i;
        if (j < d) {
#pragma clang fp contract(off)
          xs[w][j] = y[i] - us[w][j];
        }
      }
      __builtin_amdgcn_wave_barrier();
      for (int j = lane; j < d; j += 64) {
        float acc = 0.0f;
        for (int k = 0; k < d; ++k) acc = __builtin_fmaf(xs[w][k], R[(int64_t)k * d + j], acc);
        resid[v * d + j] = acc;
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// decompress: one wave per vector, x^ = clamp(((code s + lo) r) R, +-65504)
__global__ void __launch_bounds__(kGW * 64)
    group_gpu_decompress_kernel(const void *radius, const uint8_t *codes, const void *mins, const void *scales,
                                int pdt, const float *R, int64_t n, int d, int bits, int gs, void *out,
                                int out_dtype) {
  __shared__ float ys[kGW][kGMax];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int ng = (d + gs - 1) / gs, dpad = ng * gs;
  const int cb = store_bits(bits);
  const int row_bytes = dpad * cb / 8;
  for (int64_t v = (int64_t)blockIdx.x * kGW + w; v < n; v += (int64_t)gridDim.x * kGW) {
    const float r = ld_par(radius, pdt, v);
    const uint8_t *crow = codes + v * row_bytes;
    for (int j = lane; j < d; j += 64) {
#pragma clang fp contract(off)
      const int g = j / gs;
      const float dq = (float)code_at(crow, cb, j) * ld_par(scales, pdt, v * ng + g) + ld_par(mins, pdt, v * ng + g);
      ys[w][j] = dq * r;
    }
    __builtin_amdgcn_wave_barrier();
    for (int j = lane; j < d; j += 64) {
      float acc = 0.0f;
      for (int k = 0; k < d; ++k) acc = __builtin_fmaf(ys[w][k], R[(int64_t)k * d + j], acc);
      acc = acc > 65504.0f ? 65504.0f : acc < -65504.0f ? -65504.0f : acc;
      if (out_dtype == PQKV_F16) ((half_t *)out)[v * d + j] = (half_t)acc;
      else ((float *)out)[v * d + j] = acc;
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// QJL sketch: e = x (- x_hat), signs of P e (fp64 sums, P given transposed
// as Pt [d][m] fp64), LSB first, bits past m zero; norm |e| (fp64, stored in
// norm_dtype). One wave per vector.
__global__ void __launch_bounds__(kGW * 64)
    qjl_sketch_kernel(const void *x, int x_dtype, const float *x_hat, const double *Pt, int64_t n, int d, int m,
                      uint8_t *signs, void *norms, int norm_dtype) {
  __shared__ double es[kGW][kGMax];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int m8 = (m + 7) / 8;
  for (int64_t v = (int64_t)blockIdx.x * kGW + w; v < n; v += (int64_t)gridDim.x * kGW) {
    double sq = 0.0;
    for (int k = lane; k < d; k += 64) {
      float e = ld_in(x, x_dtype, v * d + k);
      if (x_hat) {
#pragma clang fp contract(off)
        e = e - x_hat[v * d + k];
      }
      es[w][k] = (double)e;
      sq += (double)e * (double)e;
    }
    for (int s = 32; s > 0; s >>= 1) sq += __shfl_xor(sq, s, 64);
    __builtin_amdgcn_wave_barrier();
    for (int i0 = 0; i0 < m; i0 += 64) {
      const int i = i0 + lane;
      double acc = 0.0;
      if (i < m)
        for (int k = 0; k < d; ++k) acc = __builtin_fma(es[w][k], Pt[(int64_t)k * m + i], acc);
      const uint64_t bal = __builtin_amdgcn_ballot_w64(i < m && acc >= 0.0);
      if (lane < 8 && i0 / 8 + lane < m8) signs[v * m8 + i0 / 8 + lane] = (uint8_t)(bal >> (8 * lane));
    }
    if (lane == 0) st_par(norms, norm_dtype, v, (float)__builtin_sqrt(sq));
    __builtin_amdgcn_wave_barrier();
  }
}

// Query preparation for the fused attention: q_rot = (R q) qs zero-padded to
// dpad and pq = (P q) qs / m (P [m][d] fp32), each output one FMA chain over
// k ascending. blockIdx.y picks a slice of 64 outputs (the dpad outputs of
// R, then the m outputs of P); the workgroup stages those 64 rows of R or P
// in LDS once, with all its loads in flight together, and its four waves
// take one query row each, lane j computing output j of the slice.
constexpr int kQRows = 64;
constexpr int kQPer = kQRows * kGMax / (kGW * 64);   // staged floats per thread
__global__ void __launch_bounds__(kGW * 64)
    group_qprep_kernel(const void *q, int q_dtype, const float *R, const float *P, int64_t rows, int d, int dpad,
                       int m, float qs, float *q_rot, float *pq) {
  __shared__ float xq[kGW][kGMax];
  __shared__ float mat[kQRows][kGMax + 1];   // row pitch 257: lane j's reads of row j hit distinct banks
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int r_slices = (dpad + kQRows - 1) / kQRows;
  const bool is_p = (int)blockIdx.y >= r_slices;
  const int j0 = (is_p ? (int)blockIdx.y - r_slices : (int)blockIdx.y) * kQRows;
  const float *M = is_p ? P : R;
  const int n = is_p ? m : min(d, dpad);      // rows of M that exist
  if (M) {
    float t[kQPer];
#pragma unroll
    for (int i = 0; i < kQPer; ++i) {
      const int e = tid + i * kGW * 64, r = e / kGMax, c = e - r * kGMax;
      t[i] = (c < d && j0 + r < n) ? M[(int64_t)(j0 + r) * d + c] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < kQPer; ++i) {
      const int e = tid + i * kGW * 64, r = e / kGMax, c = e - r * kGMax;
      mat[r][c] = t[i];
    }
  }
  const int j = j0 + lane;
  const float sc = is_p ? qs / (float)m : qs;
  for (int64_t base = (int64_t)blockIdx.x * kGW; base < rows; base += (int64_t)gridDim.x * kGW) {
    const int64_t v = base + w;
    const bool live = v < rows;
    for (int k = lane; k < d; k += 64) xq[w][k] = live ? ld_in(q, q_dtype, v * d + k) : 0.0f;
    __syncthreads();
    float acc = 0.0f;
    if (M) {
      if (j < n)
        for (int k = 0; k < d; ++k) acc = __builtin_fmaf(mat[lane][k], xq[w][k], acc);
    } else if (j < d) {
      acc = xq[w][j];
    }
    if (live) {
      if (is_p) {
        if (j < m) pq[v * m + j] = acc * sc;
      } else if (j < dpad) {
        q_rot[v * dpad + j] = (j < d ? acc : 0.0f) * sc;
      }
    }
    __syncthreads();   // xq is reused by the next rows
  }
}

// ---------------------------------------------------------------------------
// Fused split-K attention on the group format. One workgroup of 4 waves =
// one (batch, kv head, split); G query rows of the kv head (rows q_off ..
// q_off + g - 1 of its group); each wave takes 64-token chunks.
//   keys:   lane = token; the token's code words are read straight from HBM
//           (16-byte loads), each code converted to fp32 and multiplied into
//           the G rows' dots group by group, s = r sum_g (s_g dot_g +
//           lo_g qsum_g) (+ the QJL term from a 4-bit-slice table of P q);
//   softmax: online, exp2 domain, per row with wave reductions;
//   values: lane = (token group, unit of 8 codes); per token the lane adds
//           (p r s_g) c_j to its 8 coordinates and p r lo_g to a per-row sum
//           that joins every coordinate of the unit at the end.
struct GroupAttnArgs {
  const float *q;                 // [B][Hq][dpad] rotated, x scale log2(e), zero past d
  const float *pq;                // [B][Hq][m] (P q) scale log2(e) / m, or null
  const uint8_t *k_codes, *v_codes;     // [B][Hkv][S_max][row_bytes]
  const void *k_rad, *v_rad;            // [B][Hkv][S_max]
  const void *k_lo, *k_sc, *v_lo, *v_sc;   // [B][Hkv][S_max][ng]
  const uint8_t *qjl;             // [B][Hkv][S_max][m / 8] or null
  const void *res_norm;           // [B][Hkv][S_max] (QJL: 0 -> no correction) or null (all-ones rule)
  const float *tab;               // codebook mode: c[code] (tab_levels entries), one group, no lo / s
  int tab_levels;
  float *part;                    // [B][Hq][splits][d + 2]
  int B, Hq, Hkv, S, S_max, d, dpad, gs, ng, cb, pdt, m;
  int gq, q_off, g, splits, tps;
};

// CB (codebook mode, the reference kernels' SoA layout at any head dim):
// a code's value is c[code] from a 16-entry table and the whole vector is
// one group with s = 1 and lo = 0, so s_t = r_t q.c[idx_t] and o_rot =
// sum_t w_t r_t c[vidx_t] (csrc/flash_turboquant.cu:27-105).
template <int G, bool CB>
__global__ void __launch_bounds__(256) group_attn_split_kernel(const GroupAttnArgs a) {
  constexpr int GP = (G + 3) & ~3;
  extern __shared__ __align__(16) float lds[];
  __shared__ float cbl[16];
  const int dpad = a.dpad, ng = a.ng, gs = a.gs, cb = a.cb, m = a.m;
  // dynamic LDS: q [G][dpad] | qsum [G][ng] | { pr [4][64][GP] | qt [m/4][16][GP] } aliased by red_o [4][G][dpad]
  float *q_lds = lds;
  float *qsum = q_lds + G * dpad;
  float *dyn = qsum + ((G * ng + 3) & ~3);
  float *pr = dyn;
  float *qt = pr + 4 * 64 * GP;
  float *red_o = dyn;
  __shared__ float red_m[4][G], red_l[4][G];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int split = blockIdx.x, bh = blockIdx.y;
  const int b = bh / a.Hkv, h = bh - b * a.Hkv;
  const int t_begin = split * a.tps;
  const int t_end = min(a.S, t_begin + a.tps);
  const int64_t stream = (int64_t)(b * a.Hkv + h) * a.S_max;
  const int row_bytes = dpad * cb / 8;
  const int row0 = b * a.Hq + h * a.gq + a.q_off;   // first query row of this launch

  for (int i = tid; i < G * dpad; i += 256) {
    const int hh = i / dpad, j = i - hh * dpad;
    q_lds[i] = hh < a.g ? a.q[(int64_t)(row0 + hh) * dpad + j] : 0.0f;
  }
  if (CB && tid < 16) cbl[tid] = tid < a.tab_levels ? a.tab[tid] : 0.0f;   // codes past the table read 0
  __syncthreads();
  for (int i = tid; i < G * ng; i += 256) {
    const int hh = i / ng, g = i - hh * ng;
    float sacc = 0.0f;
    for (int j = 0; j < gs; ++j) sacc += q_lds[hh * dpad + g * gs + j];
    qsum[i] = sacc;
  }
  if (a.qjl) {
    // qt[p][v][hh] = sum_{j<4} (bit j of v ? +1 : -1) pq[hh][4p + j]
    for (int i = tid; i < (m / 4) * 16 * GP; i += 256) {
      const int hh = i % GP, vv = (i / GP) & 15, p = i / (16 * GP);
      float acc = 0.0f;
      if (hh < a.g) {
        const float *pqr = a.pq + (int64_t)(row0 + hh) * m + 4 * p;
#pragma unroll
        for (int j = 0; j < 4; ++j) acc += ((vv >> j) & 1) ? pqr[j] : -pqr[j];
      }
      qt[i] = acc;
    }
  }
  __syncthreads();

  float m_run[G], l_run[G], o[G][8], pm[G];
#pragma unroll
  for (int hh = 0; hh < G; ++hh) {
    m_run[hh] = -INFINITY;
    l_run[hh] = 0.0f;
    pm[hh] = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c) o[hh][c] = 0.0f;
  }
  // value lanes: unit u (codes 8u .. 8u + 7) of token group tg; U rounded
  // up to a power of two so that the token groups reduce by lane xor
  const int U = dpad / 8;
  int Up = 1;
  while (Up < U) Up <<= 1;
  const int TG = 64 / Up;
  const int vu = lane % Up, vtg = lane / Up;
  const bool vact = vu < U;
  const int vg = vact ? (8 * vu) / gs : 0;
  float *prw = pr + wave * 64 * GP;

  for (int chunk = wave;; chunk += 4) {
    const int t0 = t_begin + chunk * 64;
    if (t0 >= t_end) break;
    const int tok = t0 + lane;
    const bool valid = tok < t_end;
    const int64_t ti = stream + (valid ? tok : t_begin);
    // ---- scores: lane = token ----
    float s[G];
#pragma unroll
    for (int hh = 0; hh < G; ++hh) s[hh] = 0.0f;
    const uint8_t *krow = a.k_codes + ti * row_bytes;
    const int cpw = 32 / cb;             // codes per dword
    for (int g = 0; g < ng; ++g) {
      float dot[G];
#pragma unroll
      for (int hh = 0; hh < G; ++hh) dot[hh] = 0.0f;
      const int wd0 = g * gs / cpw, wd1 = (g + 1) * gs / cpw;
      for (int wd = wd0; wd < wd1; wd += 4) {
        const int nw = min(4, wd1 - wd);
        uint32_t wv[4];
        if (nw == 4 && (((uintptr_t)(krow + 4 * wd)) & 15) == 0) {
          const u32x4 v4 = *(const u32x4 *)(krow + 4 * wd);
          wv[0] = v4.x; wv[1] = v4.y; wv[2] = v4.z; wv[3] = v4.w;
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) wv[i] = i < nw ? *(const uint32_t *)(krow + 4 * (wd + i)) : 0u;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (i >= nw) break;
          const uint32_t w32 = wv[i];
          const int j0 = (wd + i) * cpw;
          if (cb == 4) {
            const uint32_t lo4 = w32 & 0x0F0F0F0Fu, hi4 = (w32 >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              const float c0 = cval<CB>(cbl, (lo4 >> (8 * k)) & 0xFFu), c1 = cval<CB>(cbl, (hi4 >> (8 * k)) & 0xFFu);
#pragma unroll
              for (int hh = 0; hh < G; ++hh) {
                const float2 qq = *(const float2 *)&q_lds[hh * dpad + j0 + 2 * k];
                dot[hh] = __builtin_fmaf(c0, qq.x, dot[hh]);
                dot[hh] = __builtin_fmaf(c1, qq.y, dot[hh]);
              }
            }
          } else if (cb == 2) {
#pragma unroll
            for (int k = 0; k < 16; k += 4) {
              const float c0 = cval<CB>(cbl, (w32 >> (2 * k)) & 3u), c1 = cval<CB>(cbl, (w32 >> (2 * k + 2)) & 3u);
              const float c2 = cval<CB>(cbl, (w32 >> (2 * k + 4)) & 3u), c3 = cval<CB>(cbl, (w32 >> (2 * k + 6)) & 3u);
#pragma unroll
              for (int hh = 0; hh < G; ++hh) {
                const float4 qq = *(const float4 *)&q_lds[hh * dpad + j0 + k];
                dot[hh] = __builtin_fmaf(c0, qq.x, dot[hh]);
                dot[hh] = __builtin_fmaf(c1, qq.y, dot[hh]);
                dot[hh] = __builtin_fmaf(c2, qq.z, dot[hh]);
                dot[hh] = __builtin_fmaf(c3, qq.w, dot[hh]);
              }
            }
          } else {
            const float c0 = cval<CB>(cbl, w32 & 0xFFu), c1 = cval<CB>(cbl, (w32 >> 8) & 0xFFu);
            const float c2 = cval<CB>(cbl, (w32 >> 16) & 0xFFu), c3 = cval<CB>(cbl, w32 >> 24);
#pragma unroll
            for (int hh = 0; hh < G; ++hh) {
              const float4 qq = *(const float4 *)&q_lds[hh * dpad + j0];
              dot[hh] = __builtin_fmaf(c0, qq.x, dot[hh]);
              dot[hh] = __builtin_fmaf(c1, qq.y, dot[hh]);
              dot[hh] = __builtin_fmaf(c2, qq.z, dot[hh]);
              dot[hh] = __builtin_fmaf(c3, qq.w, dot[hh]);
            }
          }
        }
      }
      if (CB) {
#pragma unroll
        for (int hh = 0; hh < G; ++hh) s[hh] += dot[hh];
      } else {
        const float sc = ld_par(a.k_sc, a.pdt, ti * ng + g), lo = ld_par(a.k_lo, a.pdt, ti * ng + g);
#pragma unroll
        for (int hh = 0; hh < G; ++hh)
          s[hh] = __builtin_fmaf(sc, dot[hh], __builtin_fmaf(lo, qsum[hh * ng + g], s[hh]));
      }
    }
    const float rk = ld_par(a.k_rad, a.pdt, ti);
#pragma unroll
    for (int hh = 0; hh < G; ++hh) s[hh] *= rk;
    if (a.qjl) {
      // + (1/m) sum_i (2 sign_i - 1) (P q)_i, none for a zero residual
      const uint8_t *sg = a.qjl + ti * (m / 8);
      bool zero_res;
      if (a.res_norm) {
        zero_res = ld_par(a.res_norm, a.pdt, ti) <= 1e-30f;
      } else {
        zero_res = true;
        for (int wd = 0; wd < m / 32; ++wd) zero_res = zero_res && *(const uint32_t *)(sg + 4 * wd) == 0xFFFFFFFFu;
      }
      if (!zero_res) {
        for (int wd = 0; wd < m / 32; ++wd) {
          const uint32_t bits = *(const uint32_t *)(sg + 4 * wd);
#pragma unroll
          for (int nb = 0; nb < 8; ++nb) {
            const float *e = qt + ((8 * wd + nb) * 16 + ((bits >> (4 * nb)) & 15)) * GP;
#pragma unroll
            for (int hh = 0; hh < G; ++hh) s[hh] += e[hh];
          }
        }
      }
    }
    const float rv = ld_par(a.v_rad, a.pdt, ti);
    float alpha[G];
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
      const float sv = valid ? s[hh] : -INFINITY;
      const float mnew = fmaxf(m_run[hh], wave_max(sv));
      // -inf safety: a row whose logits so far are all -inf keeps weight 0
      const float ref = mnew == -INFINITY ? 0.0f : mnew;
      alpha[hh] = m_run[hh] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run[hh] - ref);
      const float p = valid ? __builtin_amdgcn_exp2f(sv - ref) : 0.0f;
      l_run[hh] = l_run[hh] * alpha[hh] + p;
      m_run[hh] = mnew;
      prw[lane * GP + hh] = valid ? p * rv : 0.0f;
    }
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
      pm[hh] *= alpha[hh];
#pragma unroll
      for (int c = 0; c < 8; ++c) o[hh][c] *= alpha[hh];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- values: lane = (token group vtg, unit vu) ----
    if (vact) {
      const int ntok = min(64, t_end - t0);
      for (int t = vtg; t < ntok; t += TG) {
        const int64_t tv = stream + t0 + t;
        const uint8_t *vrow = a.v_codes + tv * row_bytes;
        float c[8];
        if (cb == 4) {
          const uint32_t w32 = *(const uint32_t *)(vrow + 4 * vu);
          const uint32_t lo4 = w32 & 0x0F0F0F0Fu, hi4 = (w32 >> 4) & 0x0F0F0F0Fu;
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            c[2 * k] = cval<CB>(cbl, (lo4 >> (8 * k)) & 0xFFu);
            c[2 * k + 1] = cval<CB>(cbl, (hi4 >> (8 * k)) & 0xFFu);
          }
        } else if (cb == 2) {
          const uint32_t w16 = *(const uint16_t *)(vrow + 2 * vu);
#pragma unroll
          for (int k = 0; k < 8; ++k) c[k] = cval<CB>(cbl, (w16 >> (2 * k)) & 3u);
        } else {
          const uint32_t w0 = *(const uint32_t *)(vrow + 8 * vu), w1 = *(const uint32_t *)(vrow + 8 * vu + 4);
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            c[k] = cval<CB>(cbl, (w0 >> (8 * k)) & 0xFFu);
            c[4 + k] = cval<CB>(cbl, (w1 >> (8 * k)) & 0xFFu);
          }
        }
        const float sc = CB ? 1.0f : ld_par(a.v_sc, a.pdt, tv * ng + vg);
        const float lo = CB ? 0.0f : ld_par(a.v_lo, a.pdt, tv * ng + vg);
        float pw[GP];
#pragma unroll
        for (int g4 = 0; g4 < GP; g4 += 4) {
          const float4 v4 = *(const float4 *)&prw[t * GP + g4];
          pw[g4] = v4.x; pw[g4 + 1] = v4.y; pw[g4 + 2] = v4.z; pw[g4 + 3] = v4.w;
        }
#pragma unroll
        for (int hh = 0; hh < G; ++hh) {
          const float ps = CB ? pw[hh] : pw[hh] * sc;
          if (!CB) pm[hh] = __builtin_fmaf(pw[hh], lo, pm[hh]);
#pragma unroll
          for (int k = 0; k < 8; ++k) o[hh][k] = __builtin_fmaf(ps, c[k], o[hh][k]);
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // ---- the lo terms join their unit's coordinates; token groups, then waves ----
#pragma unroll
  for (int hh = 0; hh < G; ++hh)
#pragma unroll
    for (int k = 0; k < 8; ++k) o[hh][k] += pm[hh];
  for (int sft = Up; sft < 64; sft <<= 1)
#pragma unroll
    for (int hh = 0; hh < G; ++hh)
#pragma unroll
      for (int k = 0; k < 8; ++k) o[hh][k] += shfl_xor_f(o[hh][k], sft);
#pragma unroll
  for (int hh = 0; hh < G; ++hh) l_run[hh] = wave_sum(l_run[hh]);
  __syncthreads();   // pr / qt are free from here: red_o aliases them
  if (vtg == 0 && vact) {
#pragma unroll
    for (int hh = 0; hh < G; ++hh)
#pragma unroll
      for (int k = 0; k < 8; ++k) red_o[(wave * G + hh) * dpad + 8 * vu + k] = o[hh][k];
  }
  if (lane == 0) {
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
      red_m[wave][hh] = m_run[hh];
      red_l[wave][hh] = l_run[hh];
    }
  }
  __syncthreads();
  for (int i = tid; i < a.g * a.d; i += 256) {
    const int hh = i / a.d, c = i - hh * a.d;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) mx = fmaxf(mx, red_m[w][hh]);
    float Lsum = 0.0f, O = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float f = red_m[w][hh] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(red_m[w][hh] - mx);
      Lsum += red_l[w][hh] * f;
      O += red_o[(w * G + hh) * dpad + c] * f;
    }
    float *dst = a.part + ((int64_t)(row0 + hh) * a.splits + split) * (a.d + 2);
    if (c == 0) {
      dst[0] = mx;
      dst[1] = Lsum;
    }
    dst[2 + c] = O;
  }
}

// Split merge for any d <= 256: one workgroup per query row; o_rot = sum_s
// w_s o_s / L, then out = o_rot R (R null: o_rot itself).
__global__ void __launch_bounds__(256) group_merge_kernel(const float *part, const float *R, void *out, int out_dtype,
                                                          int splits, int d) {
  __shared__ float wts[kMaxSplits];
  __shared__ float os[kGMax];
  __shared__ float red[4];
  __shared__ float s_mx, s_inv;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row = blockIdx.x;
  const float *p = part + row * splits * (d + 2);
  float mx = -INFINITY;
  for (int s = tid; s < splits; s += 256) mx = fmaxf(mx, p[(int64_t)s * (d + 2)]);
  mx = wave_max(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  if (tid == 0) s_mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  mx = s_mx;
  float L = 0.0f;
  for (int s = tid; s < splits; s += 256) {
    const float ms = p[(int64_t)s * (d + 2)];
    const float e = ms == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ms - mx);
    wts[s] = e;
    L = __builtin_fmaf(e, p[(int64_t)s * (d + 2) + 1], L);
  }
  L = wave_sum(L);
  __syncthreads();
  if (lane == 0) red[wave] = L;
  __syncthreads();
  if (tid == 0) {
    const float Lt = red[0] + red[1] + red[2] + red[3];
    s_inv = Lt > 0.0f ? 1.0f / Lt : 0.0f;
  }
  __syncthreads();
  for (int c = tid; c < d; c += 256) {
    float acc = 0.0f;
    for (int s = 0; s < splits; ++s) acc = __builtin_fmaf(wts[s], p[(int64_t)s * (d + 2) + 2 + c], acc);
    os[c] = acc * s_inv;
  }
  __syncthreads();
  for (int j = tid; j < d; j += 256) {
    float acc = 0.0f;
    if (R) {
      for (int k = 0; k < d; ++k) acc = __builtin_fmaf(os[k], R[(int64_t)k * d + j], acc);
    } else {
      acc = os[j];
    }
    if (out_dtype == PQKV_F16) ((half_t *)out)[row * d + j] = (half_t)acc;
    else ((float *)out)[row * d + j] = acc;
  }
}

// ---------------------------------------------------------------------------
// The reference kernels' SoA encoder at any even d <= 256 (the compat entry
// points use it for the head dims the fixed-d encoders are not built for):
// integration/polarquant-kv.patch:193-269 with blockDim = max(d, 128):
// y_j = sum_k x_k R[j][k] as one fp32 FMA chain in k order, |y|^2 by a
// pairwise tree over T slots (slot t holds y_t^2, zeros past d; step s adds
// slot t + s into slot t for s = T/2 .. 1), r = correctly rounded sqrt,
// u = y / r (IEEE) or 0 where r <= 1e-30, code = first index of the
// smallest |u - c_i| (strict <, running minimum from 1e30), two codes per
// byte (coordinate 2i low nibble). T is 128 for d <= 128 and 256 above: the
// reference's tree over a non-power-of-two block drops slots for 128 < d <
// 256, which this encoder does not reproduce. One wave per vector.
__global__ void __launch_bounds__(kGW * 64)
    encode_soa_generic_kernel(const float *x, const float *R, const float *codebook, int nl, float *radius_out,
                              uint8_t *packed_out, int64_t n, int d) {
  __shared__ float xs[kGW][kGMax];
  __shared__ uint8_t cq[kGW][kGMax];
  __shared__ float cb[16];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (threadIdx.x < 16) cb[threadIdx.x] = (int)threadIdx.x < nl ? codebook[threadIdx.x] : 0.0f;
  __syncthreads();
  for (int64_t v = (int64_t)blockIdx.x * kGW + w; v < n; v += (int64_t)gridDim.x * kGW) {
    for (int k = lane; k < d; k += 64) xs[w][k] = x[v * d + k];
    __builtin_amdgcn_wave_barrier();
    float y[kGPer];
#pragma unroll
    for (int i = 0; i < kGPer; ++i) {
      const int j = lane + 64 * i;
      float acc = 0.0f;
      if (j < d)
        for (int k = 0; k < d; ++k) acc = __builtin_fmaf(xs[w][k], R[(int64_t)j * d + k], acc);
      y[i] = acc;
    }
    float sq;
    {
#pragma clang fp contract(off)
      const float q0 = y[0] * y[0], q1 = y[1] * y[1];
      if (d > 128) {
        const float q2 = y[2] * y[2], q3 = y[3] * y[3];
        sq = (q0 + q2) + (q1 + q3);   // s = 128, then s = 64
      } else {
        sq = q0 + q1;                 // s = 64
      }
#pragma unroll
      for (int s = 32; s > 0; s >>= 1) sq = sq + shfl_down_f(sq, s);
    }
    const float r = (float)__builtin_sqrt((double)__shfl(sq, 0, 64));
    const bool nz = r > 1e-30f;
#pragma unroll
    for (int i = 0; i < kGPer; ++i) {
      const int j = lane + 64 * i;
      if (j < d) {
        const float u = nz ? __fdiv_rn(y[i], r) : 0.0f;
        int best = 0;
        float mb = 1e30f;
        for (int c = 0; c < nl; ++c) {
          const float e = fabsf(u - cb[c]);
          if (e < mb) {
            mb = e;
            best = c;
          }
        }
        cq[w][j] = (uint8_t)best;
      }
    }
    __builtin_amdgcn_wave_barrier();
    for (int i = lane; i < d / 2; i += 64)
      packed_out[v * (d / 2) + i] = (uint8_t)(cq[w][2 * i] | (cq[w][2 * i + 1] << 4));
    if (lane == 0) radius_out[v] = r;
    __builtin_amdgcn_wave_barrier();
  }
}

// Rotation of n rows at any d <= 256: y = x R^T (forward, y_j = sum_k x_k
// R[j][k]) or y = x R (inverse, sum_k x_k R[k][j]), one fp32 FMA chain per
// output in k order (the reference's loops, patch:395-437,508-544).
__global__ void __launch_bounds__(kGW * 64)
    rotate_generic_kernel(const float *x, const float *R, float *y, int64_t n, int d, int inverse) {
  __shared__ float xs[kGW][kGMax];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int64_t v = (int64_t)blockIdx.x * kGW + w; v < n; v += (int64_t)gridDim.x * kGW) {
    for (int k = lane; k < d; k += 64) xs[w][k] = x[v * d + k];
    __builtin_amdgcn_wave_barrier();
    for (int j = lane; j < d; j += 64) {
      float acc = 0.0f;
      if (inverse)
        for (int k = 0; k < d; ++k) acc = __builtin_fmaf(xs[w][k], R[(int64_t)k * d + j], acc);
      else
        for (int k = 0; k < d; ++k) acc = __builtin_fmaf(xs[w][k], R[(int64_t)j * d + k], acc);
      y[v * d + j] = acc;
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// ---------------------------------------------------------------------------
namespace {
int grid_for(int64_t n) {
  const int64_t blocks = (n + kGW - 1) / kGW;
  return (int)(blocks < 8192 ? (blocks > 0 ? blocks : 1) : 8192);
}
}  // namespace

hipError_t launch_encode_soa_generic(const float *x, const float *R, const float *codebook, int n_levels,
                                     float *radius, uint8_t *packed, int64_t n, int d, hipStream_t s) {
  if (d < 2 || d > kGMax || d % 2 || n_levels < 1 || n_levels > 16) return hipErrorInvalidValue;
  encode_soa_generic_kernel<<<grid_for(n), kGW * 64, 0, s>>>(x, R, codebook, n_levels, radius, packed, n, d);
  return hipGetLastError();
}

hipError_t launch_rotate_generic(const float *x, const float *R, float *y, int64_t n, int d, int inverse,
                                 hipStream_t s) {
  if (d < 1 || d > kGMax) return hipErrorInvalidValue;
  rotate_generic_kernel<<<grid_for(n), kGW * 64, 0, s>>>(x, R, y, n, d, inverse);
  return hipGetLastError();
}

hipError_t launch_group_gpu_compress(const void *x, int x_dtype, const float *Rt, const float *R, int64_t n, int d,
                                     int bits, int gs, void *radius, uint8_t *codes, void *mins, void *scales,
                                     int pdt, float *resid, hipStream_t s) {
  if (d < 1 || d > kGMax || gs < 1 || gs > d) return hipErrorInvalidValue;
  group_gpu_compress_kernel<<<grid_for(n), kGW * 64, 0, s>>>(x, x_dtype, Rt, R, n, d, bits, gs, radius, codes, mins,
                                                             scales, pdt, resid);
  return hipGetLastError();
}

hipError_t launch_group_gpu_decompress(const void *radius, const uint8_t *codes, const void *mins,
                                       const void *scales, int pdt, const float *R, int64_t n, int d, int bits,
                                       int gs, void *out, int out_dtype, hipStream_t s) {
  if (d < 1 || d > kGMax || gs < 1 || gs > d) return hipErrorInvalidValue;
  group_gpu_decompress_kernel<<<grid_for(n), kGW * 64, 0, s>>>(radius, codes, mins, scales, pdt, R, n, d, bits, gs,
                                                               out, out_dtype);
  return hipGetLastError();
}

hipError_t launch_qjl_sketch(const void *x, int x_dtype, const float *x_hat, const double *Pt, int64_t n, int d,
                             int m, uint8_t *signs, void *norms, int norm_dtype, hipStream_t s) {
  if (d < 1 || d > kGMax || m < 1) return hipErrorInvalidValue;
  qjl_sketch_kernel<<<grid_for(n), kGW * 64, 0, s>>>(x, x_dtype, x_hat, Pt, n, d, m, signs, norms, norm_dtype);
  return hipGetLastError();
}

hipError_t launch_group_qprep(const void *q, int q_dtype, const float *R, const float *P, int64_t rows, int d,
                              int dpad, int m, float qs, float *q_rot, float *pq, hipStream_t s) {
  if (d < 1 || d > kGMax || dpad > kGMax) return hipErrorInvalidValue;
  if (P && (m < 1 || m > kGMax)) return hipErrorInvalidValue;
  const int slices = (dpad + kQRows - 1) / kQRows + (P ? (m + kQRows - 1) / kQRows : 0);
  const int64_t per = (rows + kGW - 1) / kGW;
  const dim3 grid((unsigned)(per < 1024 ? (per > 0 ? per : 1) : 1024), (unsigned)slices);
  group_qprep_kernel<<<grid, kGW * 64, 0, s>>>(q, q_dtype, R, P, rows, d, dpad, m, qs, q_rot, pq);
  return hipGetLastError();
}

size_t group_attn_lds_bytes(int G, int dpad, int ng, int m) {
  const int GP = (G + 3) & ~3;
  const size_t head = (size_t)G * dpad + (((size_t)G * ng + 3) & ~(size_t)3);
  const size_t loop = (size_t)4 * 64 * GP + (size_t)(m / 4) * 16 * GP;
  const size_t red = (size_t)4 * G * dpad;
  return 4 * (head + (loop > red ? loop : red));
}

hipError_t launch_group_attn(const GroupAttnArgsHost &h, hipStream_t s) {
  GroupAttnArgs a;
  a.q = h.q;
  a.pq = h.pq;
  a.k_codes = h.k_codes;
  a.v_codes = h.v_codes;
  a.k_rad = h.k_rad;
  a.v_rad = h.v_rad;
  a.k_lo = h.k_lo;
  a.k_sc = h.k_sc;
  a.v_lo = h.v_lo;
  a.v_sc = h.v_sc;
  a.qjl = h.qjl;
  a.res_norm = h.res_norm;
  a.tab = h.cb;
  a.tab_levels = h.cb_levels;
  a.part = h.part;
  a.B = h.B;
  a.Hq = h.Hq;
  a.Hkv = h.Hkv;
  a.S = h.S;
  a.S_max = h.S_max;
  a.d = h.d;
  a.dpad = h.dpad;
  a.gs = h.gs;
  a.ng = h.dpad / h.gs;
  a.cb = store_bits(h.bits);
  a.pdt = h.pdt;
  a.m = h.qjl ? h.m : 0;
  a.gq = h.Hq / h.Hkv;
  a.splits = h.splits;
  a.tps = h.tps;
  const dim3 grid(h.splits, h.B * h.Hkv);
  const int n_sub = (a.gq + kMaxGroup - 1) / kMaxGroup;
  int off = 0;
  for (int i = 0; i < n_sub; ++i) {
    a.q_off = off;
    a.g = a.gq / n_sub + (i < a.gq % n_sub ? 1 : 0);
    const int G = a.g <= 1 ? 1 : a.g <= 2 ? 2 : a.g <= 4 ? 4 : 8;
    const size_t lds = group_attn_lds_bytes(G, a.dpad, a.ng, a.m);
#define PQKV_GA(GG)                                                                        \
  (a.tab ? (void)group_attn_split_kernel<GG, true><<<grid, 256, lds, s>>>(a)                    \
        : (void)group_attn_split_kernel<GG, false><<<grid, 256, lds, s>>>(a))
    switch (G) {
      case 1: PQKV_GA(1); break;
      case 2: PQKV_GA(2); break;
      case 4: PQKV_GA(4); break;
      default: PQKV_GA(8); break;
    }
#undef PQKV_GA
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    off += a.g;
  }
  return hipSuccess;
}

hipError_t launch_group_merge(const float *part, const float *R, void *out, int out_dtype, int64_t rows, int splits,
                              int d, hipStream_t s) {
  if (splits < 1 || splits > kMaxSplits || d > kGMax || rows < 1) return hipErrorInvalidValue;
  group_merge_kernel<<<(unsigned)rows, 256, 0, s>>>(part, R, out, out_dtype, splits, d);
  return hipGetLastError();
}

}  // namespace pqkv
