// Rotation, bit-exact quantiser, exact fused encoder and layout converters.
//
// Arithmetic contract (the reference's encode kernel, csrc/flash_turboquant.cu
// :111-175, and its ggml copy, integration/polarquant-kv.patch:193-269):
//   rot[j]  = fp32 FMA chain over k = 0..d-1 of x[k] * R[j][k]
//   radius  = sqrtf of the 128-slot shared-memory tree of rot[j]^2
//   dir[j]  = rot[j] / radius (IEEE), 0 when radius <= 1e-30
//   code[j] = first i minimising |dir[j] - c[i]|
// The tree maps onto a wave64 as lane t = slot t: the s = 64 step is done in
// lane (x[t]^2 + x[t+64]^2), the remaining steps are shuffle-downs. The file
// is compiled without FP contraction inside the quantiser so squares and adds
// round separately, as in the reference.
#include "pqkv_cells.h"
#include "pqkv_device.h"
#include "pqkv_launch.h"

namespace pqkv {

// ---------------------------------------------------------------------------
// Per-wave quantiser of one vector held as lane t -> (x0 = y[t], x1 = y[t+64])
// for D = 128, or x0 = y[t] for D = 64. Returns the fp32 radius (all lanes)
// and this lane's two codes; nl <= 16 levels, strict '<' scan. With TABLE the
// index comes from the switch-point cell table (cells, built for cb), and the
// direction from the Markstein quotient where the radius allows it: the same
// indices with one division per vector instead of one per coordinate and a
// table read instead of the scan.
// ---------------------------------------------------------------------------
template <int D, bool TABLE = false>
__device__ __forceinline__ float quantize_wave(float x0, float x1, const float *cb, int nl, int *c0, int *c1,
                                               const uint2 *cells = nullptr) {
#pragma clang fp contract(off)
  float v = x0 * x0;
  if (D == 128) {
    float w = x1 * x1;
    v = v + w;            // tree step s = 64
  }
#pragma unroll
  for (int s = 32; s > 0; s >>= 1) v = v + shfl_down_f(v, s);
  // Correctly rounded fp32 square root: v_sqrt_f32 alone is only within
  // 1 ulp, so take the fp64 root (correctly rounded) and round once to fp32,
  // which gives the correctly rounded fp32 root of an fp32 argument.
  const float r = (float)__builtin_sqrt((double)__shfl(v, 0, kWave));
  if constexpr (TABLE) {
    float d0, d1;
    if (markstein_radius(r)) {
      const float inv = r > 1e-30f ? __fdiv_rn(1.0f, r) : 0.0f;
      d0 = dir_markstein(x0, r, inv);
      d1 = dir_markstein(x1, r, inv);
    } else {
      d0 = dir_divided(x0, r);
      d1 = dir_divided(x1, r);
    }
    *c0 = table_code(cells, d0);
    *c1 = D == 128 ? table_code(cells, d1) : 0;
    return r;
  }
  const bool nz = r > 1e-30f;
  const float d0 = nz ? __fdiv_rn(x0, r) : 0.0f;
  const float d1 = nz ? __fdiv_rn(x1, r) : 0.0f;
  int b0 = 0, b1 = 0;
  float m0 = 1e30f, m1 = 1e30f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    if (i < nl) {
      const float c = cb[i];
      float e0 = fabsf(d0 - c);
      if (e0 < m0) { m0 = e0; b0 = i; }
      float e1 = fabsf(d1 - c);
      if (e1 < m1) { m1 = e1; b1 = i; }
    }
  }
  *c0 = b0;
  *c1 = b1;
  return r;
}

// Pack the wave's codes into one block_pq4 / block_pq2 vector.
template <int D, int BITS>
__device__ __forceinline__ void store_blocks_wave(int b0, int b1, float r, uint8_t *out_vec) {
  const int lane = threadIdx.x & (kWave - 1);
  const int cv = b0 | (b1 << 4);
  const uint16_t r16 = radius_half_bits(r);
  if (BITS == 4) {
    // qs byte p holds coordinates 2p (low nibble) and 2p+1 (high nibble).
    const int a = (2 * lane) & 63;
    const int va = __shfl(cv, a, kWave), vb = __shfl(cv, a + 1, kWave);
    const int sh = (D == 128 && lane >= 32) ? 4 : 0;
    const uint8_t byte = (uint8_t)(((va >> sh) & 15) | (((vb >> sh) & 15) << 4));
    if (lane < D / 2) {
      out_vec[qs_offset(lane, 4)] = byte;
      if ((lane & 15) == 0) *(uint16_t *)(out_vec + (lane >> 4) * kPq4BlockBytes) = r16;
    }
  } else {
    // qs byte p holds coordinates 4p .. 4p+3, two bits each, lowest first.
    const int a = (4 * lane) & 63;
    const int sh = (D == 128 && lane >= 16) ? 4 : 0;
    int byte = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) byte |= ((__shfl(cv, a + k, kWave) >> sh) & 3) << (2 * k);
    if (lane < D / 4) {
      out_vec[qs_offset(lane, 2)] = (uint8_t)byte;
      if ((lane & 7) == 0) *(uint16_t *)(out_vec + (lane >> 3) * kPq2BlockBytes) = r16;
    }
  }
}

// Reference SoA output: packed[p] = code(2p) | code(2p+1) << 4 for any level
// count (csrc/flash_turboquant.cu:173), fp32 radius.
template <int D>
__device__ __forceinline__ void store_soa_wave(int b0, int b1, float r, uint8_t *packed, float *radius) {
  const int lane = threadIdx.x & (kWave - 1);
  const int cv = b0 | (b1 << 4);
  const int a = (2 * lane) & 63;
  const int va = __shfl(cv, a, kWave), vb = __shfl(cv, a + 1, kWave);
  const int sh = (D == 128 && lane >= 32) ? 4 : 0;
  if (lane < D / 2) packed[lane] = (uint8_t)(((va >> sh) & 15) | (((vb >> sh) & 15) << 4));
  if (lane == 0) *radius = r;
}

template <int D, int BITS, bool TABLE = false>
__device__ __forceinline__ void quantize_store_wave(float x0, float x1, const float *cb, uint8_t *out_vec,
                                                    float *radius_out, float *r_f32, uint32_t *codes,
                                                    const uint2 *cells = nullptr) {
  int b0, b1;
  const float r = quantize_wave<D, TABLE>(x0, x1, cb, 1 << BITS, &b0, &b1, cells);
  store_blocks_wave<D, BITS>(b0, b1, r, out_vec);
  *r_f32 = r;
  *codes = (uint32_t)(b0 | (b1 << 4));
  if (radius_out != nullptr && (threadIdx.x & 63) == 0) *radius_out = r;
}

// One wave per vector; fp32 rotated input.
template <int D, int BITS>
__global__ void __launch_bounds__(256) quantize_rotated_kernel(const float *__restrict__ x_rot,
                                                               const float *__restrict__ codebook,
                                                               uint8_t *__restrict__ blocks,
                                                               float *__restrict__ radius_out,
                                                               int64_t n) {
  __shared__ float cb[16];
  if (threadIdx.x < (1 << BITS)) cb[threadIdx.x] = codebook[threadIdx.x];
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int64_t waves = (int64_t)gridDim.x * (blockDim.x / kWave);
  for (int64_t v = (int64_t)blockIdx.x * (blockDim.x / kWave) + (threadIdx.x >> 6); v < n; v += waves) {
    const float *xv = x_rot + v * D;
    const float x0 = xv[lane];
    const float x1 = D == 128 ? xv[lane + 64] : 0.0f;
    float r;
    uint32_t codes;
    quantize_store_wave<D, BITS>(x0, x1, cb, blocks + v * vector_bytes(D, BITS),
                                 radius_out ? radius_out + v : nullptr, &r, &codes);
  }
}

// ---------------------------------------------------------------------------
// Rotation: thread j of a vector group keeps row j (forward) or column j
// (inverse) of R in registers; x comes from LDS (broadcast reads).
// y[j] = fma chain over k ascending, then optional scale and dtype cast.
// ---------------------------------------------------------------------------
template <int D, bool INVERSE>
__device__ __forceinline__ void load_r_row(const float *__restrict__ R, int j, float (&rr)[D]) {
#pragma unroll
  for (int k = 0; k < D; ++k) rr[k] = INVERSE ? R[k * D + j] : R[j * D + k];
}

template <typename T>
__device__ __forceinline__ float load_as_float(const T *p) { return (float)*p; }
__device__ __forceinline__ float load_as_float(const bf16_t *p) { return bf16_to_float(p->bits); }

// y = R x (forward) or R^T x (inverse) for n vectors, each output one fp32
// FMA chain over k ascending (the encoder's order, so both agree bit for bit).
// Workgroup (vg, cg): 8 vectors x 32 output columns, one output per thread.
// The 32 rows (forward) or columns (inverse) of R it needs are staged in LDS
// as [32][D + 4]: the chain reads 16 bytes of x and of R per 4 steps, and
// with the 4-float pad each 16-lane phase of those reads covers all 64 banks.
constexpr int kRotVec = 8;   // vectors per workgroup iteration
constexpr int kRotCols = 32; // output columns per workgroup

// The vectors come from a source functor: element j of vector v.
template <typename TIN, int D>
struct PlainSource {
  const TIN *x;
  __device__ __forceinline__ float operator()(int64_t v, int j) const { return load_as_float(x + v * D + j); }
};
// fp32 rows of a strided [n_seq][Hq][n_q] arrangement read in
// [n_seq][n_q][Hq] order (ggml's flash-attn-ext query: element strides s_q
// between query rows, s_h between heads, s_s between sequences).
struct RowsSource {
  const float *x;
  int64_t s_q, s_h, s_s;
  int n_q, Hq;
  __device__ __forceinline__ float operator()(int64_t v, int j) const {
    const int64_t rest = v / Hq, h = v - rest * Hq;
    const int64_t sq = rest / n_q, iq = rest - sq * n_q;
    return x[sq * s_s + h * s_h + iq * s_q + j];
  }
};
// Block-encoded vectors (block_pq4 / block_pq2): r16 * c[code], the rotated
// reconstruction the attention kernels use.
template <int D, int BITS>
struct BlockSource {
  const uint8_t *blocks;
  const float *cb;
  __device__ __forceinline__ float operator()(int64_t v, int j) const {
    constexpr int VB = vector_bytes(D, BITS);
    const uint8_t *vec = blocks + v * VB;
    const float r = half_bits_to_float(*(const uint16_t *)vec);
    const int per = 8 / BITS;                              // codes per byte
    const uint8_t byte = vec[qs_offset(j / per, BITS)];
    const int code = (byte >> (BITS * (j % per))) & ((1 << BITS) - 1);
    return r * cb[code];
  }
};

// SAT16: fp16 output saturates at +-65504 like the reference's decompress
// (decompress_kernel.py:52-55, clamp(-65504, 65504).half()).
template <int D, bool INVERSE, typename SRC, typename TOUT, bool SAT16 = false>
__global__ void __launch_bounds__(256) rotate_kernel(const SRC src, const float *__restrict__ R,
                                                     TOUT *__restrict__ y, int64_t n, float out_scale) {
  constexpr int RP = D + 4;
  __shared__ __align__(16) float rs[kRotCols * RP];
  __shared__ __align__(16) float xs[kRotVec * D];
  const int tid = threadIdx.x;
  const int c0 = blockIdx.y * kRotCols;
  // The first group's vector loads go out before the R staging loads, so
  // the two global round trips overlap.
  constexpr int XU = kRotVec * D / 256;
  const int64_t stride = (int64_t)gridDim.x * kRotVec;
  float xv[XU];
  auto load_x = [&](int64_t bs) {
#pragma unroll
    for (int u = 0; u < XU; ++u) {
      const int i = tid + 256 * u;
      const int64_t v = bs + i / D;
      xv[u] = v < n ? src(v, i % D) : 0.0f;
    }
  };
  load_x((int64_t)blockIdx.x * kRotVec);
  // rs[jj][k] = R[c0 + jj][k] (forward) or R[k][c0 + jj] (inverse)
  if (!INVERSE) {
#pragma unroll
    for (int u = 0; u < kRotCols * D / 4 / 256; ++u) {
      const int i = tid + 256 * u, jj = i / (D / 4), k4 = i % (D / 4);
      *(float4 *)(rs + jj * RP + 4 * k4) = *(const float4 *)(R + (int64_t)(c0 + jj) * D + 4 * k4);
    }
  } else {
#pragma unroll
    for (int u = 0; u < kRotCols * D / 4 / 256; ++u) {
      const int i = tid + 256 * u, k = i / (kRotCols / 4), j4 = i % (kRotCols / 4);
      const float4 v = *(const float4 *)(R + (int64_t)k * D + c0 + 4 * j4);
      rs[(4 * j4 + 0) * RP + k] = v.x;
      rs[(4 * j4 + 1) * RP + k] = v.y;
      rs[(4 * j4 + 2) * RP + k] = v.z;
      rs[(4 * j4 + 3) * RP + k] = v.w;
    }
  }
  const int jj = tid % kRotCols, g = tid / kRotCols;   // g: vector of the group
  for (int64_t base = (int64_t)blockIdx.x * kRotVec; base < n; base += stride) {
#pragma unroll
    for (int u = 0; u < XU; ++u) xs[tid + 256 * u] = xv[u];
    __syncthreads();
    if (base + stride < n) load_x(base + stride);
    const float4 *xr = (const float4 *)(xs + g * D);
    const float4 *rr = (const float4 *)(rs + jj * RP);
    float acc = 0.0f;
#pragma unroll 4
    for (int k4 = 0; k4 < D / 4; ++k4) {
      const float4 a4 = xr[k4], r4 = rr[k4];
      acc = __builtin_fmaf(a4.x, r4.x, acc);
      acc = __builtin_fmaf(a4.y, r4.y, acc);
      acc = __builtin_fmaf(a4.z, r4.z, acc);
      acc = __builtin_fmaf(a4.w, r4.w, acc);
    }
    const int64_t v = base + g;
    if (v < n) {
      float o = acc * out_scale;
      if (SAT16) o = o > 65504.0f ? 65504.0f : (o < -65504.0f ? -65504.0f : o);
      y[v * D + c0 + jj] = (TOUT)o;
    }
    __syncthreads();
  }
}

// The identity rotation: y = x * out_scale (what rotate_kernel gives for
// R = I, whose FMA chain adds exact zeros to x_j * 1).
template <typename TIN, typename TOUT>
__global__ void __launch_bounds__(256) scale_kernel(const TIN *__restrict__ x, TOUT *__restrict__ y, int64_t n,
                                                    float out_scale) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    y[i] = (TOUT)(load_as_float(x + i) * out_scale);
}

// Two chained forward rotations in one launch: y = (R x) sy, then
// z = (M y) sz (decode with QJL: the rotated query and its projections
// P_rot q_rot / m). Workgroup: kRot2Vec vectors, all D columns, both
// matrices staged whole in LDS ([D][D + 4], padded for 16-byte reads) by one
// round of loads.
// Every output is the FMA chain of rotate_kernel over k ascending, so y and
// z are bit-identical to two rotate_kernel launches.
constexpr int kRot2Vec = 2;
template <int D, typename TIN>
__global__ void __launch_bounds__(256) rotate2_kernel(const TIN *__restrict__ x, const float *__restrict__ R,
                                                      const float *__restrict__ M, float *__restrict__ y,
                                                      float *__restrict__ z, int64_t n, float sy, float sz) {
  constexpr int RP = D + 4;
  constexpr int NO = kRot2Vec * D;  // outputs per matrix
  __shared__ __align__(16) float rs[D * RP];
  __shared__ __align__(16) float ms[D * RP];
  __shared__ __align__(16) float xs[NO];
  __shared__ __align__(16) float ys[NO];
  const int tid = threadIdx.x;
  const int64_t base = (int64_t)blockIdx.x * kRot2Vec;
  for (int i = tid; i < NO; i += 256) {
    const int64_t v = base + i / D;
    xs[i] = v < n ? load_as_float(x + v * D + (i % D)) : 0.0f;
  }
#pragma unroll 4
  for (int i = tid; i < D * D / 4; i += 256) {
    const int j = i / (D / 4), k4 = i % (D / 4);
    const float4 a = *(const float4 *)(R + (int64_t)j * D + 4 * k4);
    const float4 b = *(const float4 *)(M + (int64_t)j * D + 4 * k4);
    *(float4 *)(rs + j * RP + 4 * k4) = a;
    *(float4 *)(ms + j * RP + 4 * k4) = b;
  }
  __syncthreads();
  for (int i = tid; i < NO; i += 256) {
    const int g = i / D, j = i % D;
    const float4 *ar = (const float4 *)(xs + g * D), *mr = (const float4 *)(rs + j * RP);
    float acc = 0.0f;
#pragma unroll 4
    for (int k4 = 0; k4 < D / 4; ++k4) {
      const float4 a4 = ar[k4], m4 = mr[k4];
      acc = __builtin_fmaf(a4.x, m4.x, acc);
      acc = __builtin_fmaf(a4.y, m4.y, acc);
      acc = __builtin_fmaf(a4.z, m4.z, acc);
      acc = __builtin_fmaf(a4.w, m4.w, acc);
    }
    const float yv = acc * sy;
    ys[i] = yv;
    if (base + g < n) y[(base + g) * D + j] = yv;
  }
  __syncthreads();
  for (int i = tid; i < NO; i += 256) {
    const int g = i / D, j = i % D;
    const float4 *ar = (const float4 *)(ys + g * D), *mr = (const float4 *)(ms + j * RP);
    float acc = 0.0f;
#pragma unroll 4
    for (int k4 = 0; k4 < D / 4; ++k4) {
      const float4 a4 = ar[k4], m4 = mr[k4];
      acc = __builtin_fmaf(a4.x, m4.x, acc);
      acc = __builtin_fmaf(a4.y, m4.y, acc);
      acc = __builtin_fmaf(a4.z, m4.z, acc);
      acc = __builtin_fmaf(a4.w, m4.w, acc);
    }
    if (base + g < n) z[(base + g) * D + j] = acc * sz;
  }
}

hipError_t launch_rotate2(const void *x, int x_dtype, const float *R, const float *M, float *y, float *z, int64_t n,
                          int d, float sy, float sz, hipStream_t s) {
  const int64_t grid = (n + kRot2Vec - 1) / kRot2Vec;
  if (grid < 1 || grid > 0x7fffffff) return hipErrorInvalidValue;
  if (d == 128) {
    if (x_dtype == 0) rotate2_kernel<128, float><<<(int)grid, 256, 0, s>>>((const float *)x, R, M, y, z, n, sy, sz);
    else rotate2_kernel<128, half_t><<<(int)grid, 256, 0, s>>>((const half_t *)x, R, M, y, z, n, sy, sz);
  } else {
    if (x_dtype == 0) rotate2_kernel<64, float><<<(int)grid, 256, 0, s>>>((const float *)x, R, M, y, z, n, sy, sz);
    else rotate2_kernel<64, half_t><<<(int)grid, 256, 0, s>>>((const half_t *)x, R, M, y, z, n, sy, sz);
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Exact fused encoders: the rotation above (bit-identical FMA chain) followed
// by the per-wave quantiser. 256 threads; a tile is EV = kExactChains *
// (256 / D) vectors. Thread (j, g) = (tid % D, tid / D) keeps row j of R in
// registers and runs kExactChains independent chains, for vectors g,
// g + 256 / D, ... of the tile, each over k ascending: the arithmetic of one
// chain per vector, with several chains' latencies overlapped in a thread.
// Each wave then quantises EV / 4 of the tile's vectors. The next tile's
// inputs are loaded into registers while this one is rotated.
// ---------------------------------------------------------------------------
constexpr int kExactChains = 4;

template <int D>
struct ExactTile {
  static constexpr int TG = 256 / D;              // threads per output coordinate
  static constexpr int EV = TG * kExactChains;    // vectors per tile
  static constexpr int QW = EV / 4;               // vectors each wave quantises
};

// The tile's rotation: ys[t][j] = FMA chain over k of xs[t][k] R[j][k] for
// t = g + TG i.
template <int D>
__device__ __forceinline__ void rotate_tile(const float (*xs)[D], float (*ys)[D + 1], const float (&rr)[D], int j,
                                            int g) {
  constexpr int TG = ExactTile<D>::TG;
  float acc[kExactChains];
#pragma unroll
  for (int i = 0; i < kExactChains; ++i) acc[i] = 0.0f;
#pragma unroll
  for (int k4 = 0; k4 < D / 4; ++k4) {
#pragma unroll
    for (int i = 0; i < kExactChains; ++i) {
      const float4 x4 = *(const float4 *)&xs[g + TG * i][4 * k4];
      acc[i] = __builtin_fmaf(x4.x, rr[4 * k4], acc[i]);
      acc[i] = __builtin_fmaf(x4.y, rr[4 * k4 + 1], acc[i]);
      acc[i] = __builtin_fmaf(x4.z, rr[4 * k4 + 2], acc[i]);
      acc[i] = __builtin_fmaf(x4.w, rr[4 * k4 + 3], acc[i]);
    }
  }
#pragma unroll
  for (int i = 0; i < kExactChains; ++i) ys[g + TG * i][j] = acc[i];
}

// block_pq4 / block_pq2 output (strided, paged), fp32 or fp16 input, plus
// the optional QJL sign sketch.
template <int D, int BITS, typename TIN>
__global__ void __launch_bounds__(256) encode_exact_kernel(EncodeArgs a) {
  constexpr int TG = ExactTile<D>::TG, EV = ExactTile<D>::EV, QW = ExactTile<D>::QW;
  constexpr int VB = vector_bytes(D, BITS);
  __shared__ __align__(16) float xs[EV][D];
  __shared__ float ys[EV][D + 1];
  __shared__ float rs[EV];
  __shared__ uint32_t cs[EV][64];
  __shared__ float cb[16], thr[16];
  __shared__ int ucell[16];
  __shared__ int table_ok;
  __shared__ uint2 cells[kECellSlots];
  const int tid = threadIdx.x;
  const int j = tid % D, g = tid / D;
  const int lane = tid & 63, wave = tid >> 6;
  if (tid < 16) cb[tid] = tid < (1 << BITS) ? a.codebook[tid] : 0.0f;
  __syncthreads();
  build_cell_table(cb, 1 << BITS, tid, cells, thr, ucell, &table_ok);
  const bool use_table = table_ok != 0;
  float rr[D];
  load_r_row<D, false>(a.R, j, rr);
  const TIN *x = (const TIN *)a.x;
  const int64_t n = a.n_outer * a.n_inner;
  const int64_t stride = (int64_t)gridDim.x * EV;
  const bool qjl = a.qjl != nullptr || a.qjl_pages != nullptr;
  float xv[kExactChains];
  auto load_x = [&](int64_t base) {
#pragma unroll
    for (int i = 0; i < kExactChains; ++i) {
      const int64_t v = base + g + TG * i;
      float t = 0.0f;
      if (v < n) {
        const int64_t vo = v / a.n_inner, vi = v - vo * a.n_inner;
        t = load_as_float(x + vo * a.x_outer_stride + vi * D + j);
      }
      xv[i] = t;
    }
  };
  load_x((int64_t)blockIdx.x * EV);
  for (int64_t base = (int64_t)blockIdx.x * EV; base < n; base += stride) {
#pragma unroll
    for (int i = 0; i < kExactChains; ++i) xs[g + TG * i][j] = xv[i];
    __syncthreads();
    if (base + stride < n) load_x(base + stride);
    rotate_tile<D>(xs, ys, rr, j, g);
    __syncthreads();
    // Quantise: wave w handles vectors QW w .. QW w + QW - 1 of the tile.
#pragma unroll
    for (int q = 0; q < QW; ++q) {
      const int t = QW * wave + q;
      const int64_t qv = base + t;
      if (qv < n) {
        const int64_t qo = qv / a.n_inner, qi = qv - qo * a.n_inner;
        const float x0 = ys[t][lane];
        const float x1 = D == 128 ? ys[t][lane + 64] : 0.0f;
        float r;
        uint32_t codes;
        uint8_t *out = encode_out_addr(a, a.blocks, a.pages, a.blocks_outer_stride, qo, qi, VB);
        if (use_table) quantize_store_wave<D, BITS, true>(x0, x1, cb, out, nullptr, &r, &codes, cells);
        else quantize_store_wave<D, BITS>(x0, x1, cb, out, nullptr, &r, &codes);
        cs[t][lane] = codes;
        if (lane == 0) rs[t] = r;
      }
    }
    if (qjl) {
      __syncthreads();
      // Residual e = y - r * c[code] in LDS (overwrites xs), then sign of
      // p_rot[i] . e for i = j (m = D projections, one per thread).
#pragma unroll
      for (int i = 0; i < kExactChains; ++i) {
        const int t = g + TG * i;
        if (base + t < n) {
          const uint32_t cw = cs[t][j & 63];
          const int code = D == 128 ? ((j < 64) ? (cw & 15) : (cw >> 4)) : (cw & 15);
          xs[t][j] = ys[t][j] - rs[t] * cb[code];
        }
      }
      __syncthreads();
      float proj[kExactChains];
#pragma unroll
      for (int i = 0; i < kExactChains; ++i) proj[i] = 0.0f;
#pragma unroll 8
      for (int k = 0; k < D; ++k) {
        const float pk = a.p_rot[j * D + k];
#pragma unroll
        for (int i = 0; i < kExactChains; ++i) proj[i] = __builtin_fmaf(pk, xs[g + TG * i][k], proj[i]);
      }
#pragma unroll
      for (int i = 0; i < kExactChains; ++i) {
        const int64_t v = base + g + TG * i;
        const uint64_t bits = __ballot(proj[i] >= 0.0f);
        if (v < n && lane == 0) {
          const int64_t qo = v / a.n_inner, qi = v - qo * a.n_inner;
          *(uint64_t *)(encode_out_addr(a, a.qjl, a.qjl_pages, a.qjl_outer_stride, qo, qi, D / 8) + (j / 64) * 8) =
              bits;
        }
      }
    }
    __syncthreads();
  }
}

// Reference-format encoder (fp32 input, SoA output, any level count <= 16):
// the exact rotation and quantiser above, written as packed nibbles plus fp32
// radius, i.e. the output of turboquant_compress_kernel.
template <int D>
__global__ void __launch_bounds__(256) encode_soa_kernel(const float *__restrict__ x, const float *__restrict__ R,
                                                         const float *__restrict__ codebook, int nl,
                                                         float *__restrict__ radius_out,
                                                         uint8_t *__restrict__ packed_out, int64_t n) {
  constexpr int TG = ExactTile<D>::TG, EV = ExactTile<D>::EV, QW = ExactTile<D>::QW;
  __shared__ __align__(16) float xs[EV][D];
  __shared__ float ys[EV][D + 1];
  __shared__ float cb[16], thr[16];
  __shared__ int ucell[16];
  __shared__ int table_ok;
  __shared__ uint2 cells[kECellSlots];
  const int tid = threadIdx.x;
  const int j = tid % D, g = tid / D;
  const int lane = tid & 63, wave = tid >> 6;
  if (tid < 16) cb[tid] = tid < nl ? codebook[tid] : 0.0f;
  __syncthreads();
  build_cell_table(cb, nl, tid, cells, thr, ucell, &table_ok);
  const bool use_table = table_ok != 0;
  float rr[D];
  load_r_row<D, false>(R, j, rr);
  const int64_t stride = (int64_t)gridDim.x * EV;
  float xv[kExactChains];
  auto load_x = [&](int64_t base) {
#pragma unroll
    for (int i = 0; i < kExactChains; ++i) {
      const int64_t v = base + g + TG * i;
      xv[i] = v < n ? x[v * D + j] : 0.0f;
    }
  };
  load_x((int64_t)blockIdx.x * EV);
  for (int64_t base = (int64_t)blockIdx.x * EV; base < n; base += stride) {
#pragma unroll
    for (int i = 0; i < kExactChains; ++i) xs[g + TG * i][j] = xv[i];
    __syncthreads();
    if (base + stride < n) load_x(base + stride);
    rotate_tile<D>(xs, ys, rr, j, g);
    __syncthreads();
#pragma unroll
    for (int q = 0; q < QW; ++q) {
      const int t = QW * wave + q;
      const int64_t qv = base + t;
      if (qv < n) {
        int b0, b1;
        const float y0 = ys[t][lane], y1 = D == 128 ? ys[t][lane + 64] : 0.0f;
        const float r = use_table ? quantize_wave<D, true>(y0, y1, cb, nl, &b0, &b1, cells)
                                  : quantize_wave<D>(y0, y1, cb, nl, &b0, &b1);
        store_soa_wave<D>(b0, b1, r, packed_out + qv * (D / 2), radius_out + qv);
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// SoA (packed u8 [n][d/2] + f32 radius [n]) <-> block_pq4.
// ---------------------------------------------------------------------------
__global__ void soa_to_blocks_kernel(const uint8_t *__restrict__ packed, const float *__restrict__ radius,
                                     uint8_t *__restrict__ blocks, int64_t n, int d) {
  const int64_t per = d / 2 + d / 32;  // qs bytes + radius halves per vector
  const int64_t total = n * per;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t v = t / per;
    const int e = (int)(t - v * per);
    uint8_t *dst = blocks + v * (int64_t)vector_bytes(d, 4);
    if (e < d / 2) {
      dst[qs_offset(e, 4)] = packed[v * (d / 2) + e];
    } else {
      const int b = e - d / 2;
      *(uint16_t *)(dst + b * kPq4BlockBytes) = radius_half_bits(radius[v]);
    }
  }
}

__global__ void blocks_to_soa_kernel(const uint8_t *__restrict__ blocks, uint8_t *__restrict__ packed,
                                     float *__restrict__ radius, int64_t n, int d) {
  const int64_t per = d / 2 + 1;
  const int64_t total = n * per;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t v = t / per;
    const int e = (int)(t - v * per);
    const uint8_t *src = blocks + v * (int64_t)vector_bytes(d, 4);
    if (e < d / 2) packed[v * (d / 2) + e] = src[qs_offset(e, 4)];
    else radius[v] = half_bits_to_float(*(const uint16_t *)src);
  }
}

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------
static int grid_for(int64_t items, int per_block, int cap = 8192) {
  int64_t g = (items + per_block - 1) / per_block;
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return (int)g;
}

hipError_t launch_quantize_rotated(const float *x_rot, const float *codebook, int bits, uint8_t *blocks,
                                   float *radius_out, int64_t n, int d, hipStream_t s) {
  const int grid = grid_for(n, 4);
#define PQKV_QR(DD, BB) \
  quantize_rotated_kernel<DD, BB><<<grid, 256, 0, s>>>(x_rot, codebook, blocks, radius_out, n)
  if (d == 128 && bits == 4) PQKV_QR(128, 4);
  else if (d == 128 && bits == 2) PQKV_QR(128, 2);
  else if (d == 64 && bits == 4) PQKV_QR(64, 4);
  else PQKV_QR(64, 2);
#undef PQKV_QR
  return hipGetLastError();
}

template <int D, bool INV>
static void rotate_dispatch(const void *x, int xt, const float *R, void *y, int yt, int64_t n, float sc,
                            hipStream_t s) {
  const dim3 grid(grid_for(n, kRotVec, 2048), D / kRotCols);
  using F = PlainSource<float, D>;
  using H = PlainSource<half_t, D>;
  if (xt == 0 && yt == 0)
    rotate_kernel<D, INV, F, float><<<grid, 256, 0, s>>>(F{(const float *)x}, R, (float *)y, n, sc);
  else if (xt == 0 && yt == 1)
    rotate_kernel<D, INV, F, half_t><<<grid, 256, 0, s>>>(F{(const float *)x}, R, (half_t *)y, n, sc);
  else if (xt == 1 && yt == 0)
    rotate_kernel<D, INV, H, float><<<grid, 256, 0, s>>>(H{(const half_t *)x}, R, (float *)y, n, sc);
  else
    rotate_kernel<D, INV, H, half_t><<<grid, 256, 0, s>>>(H{(const half_t *)x}, R, (half_t *)y, n, sc);
}

hipError_t launch_rotate_rows(const float *x, int64_t s_q, int64_t s_h, int64_t s_s, int n_q, int Hq, int n_seq,
                              const float *R, float *y, int d, float out_scale, hipStream_t s) {
  const int64_t n = (int64_t)n_seq * n_q * Hq;
  const RowsSource src{x, s_q, s_h, s_s, n_q, Hq};
  if (d == 128) {
    const dim3 grid(grid_for(n, kRotVec, 2048), 128 / kRotCols);
    rotate_kernel<128, false, RowsSource, float><<<grid, 256, 0, s>>>(src, R, y, n, out_scale);
  } else {
    const dim3 grid(grid_for(n, kRotVec, 2048), 64 / kRotCols);
    rotate_kernel<64, false, RowsSource, float><<<grid, 256, 0, s>>>(src, R, y, n, out_scale);
  }
  return hipGetLastError();
}

template <int D, int BITS>
static void dequant_dispatch(const uint8_t *blocks, const float *cb, const float *R, void *y, int yt, int64_t n,
                             hipStream_t s) {
  const dim3 grid(grid_for(n, kRotVec, 4096), D / kRotCols);
  using S = BlockSource<D, BITS>;
  if (yt == 0) rotate_kernel<D, true, S, float><<<grid, 256, 0, s>>>(S{blocks, cb}, R, (float *)y, n, 1.0f);
  else rotate_kernel<D, true, S, half_t, true><<<grid, 256, 0, s>>>(S{blocks, cb}, R, (half_t *)y, n, 1.0f);
}

hipError_t launch_dequantize(const uint8_t *blocks, const float *codebook, int bits, const float *R, void *y,
                             int y_dtype, int64_t n, int d, hipStream_t s) {
  if (d == 128 && bits == 4) dequant_dispatch<128, 4>(blocks, codebook, R, y, y_dtype, n, s);
  else if (d == 128) dequant_dispatch<128, 2>(blocks, codebook, R, y, y_dtype, n, s);
  else if (bits == 4) dequant_dispatch<64, 4>(blocks, codebook, R, y, y_dtype, n, s);
  else dequant_dispatch<64, 2>(blocks, codebook, R, y, y_dtype, n, s);
  return hipGetLastError();
}

hipError_t launch_rotate(const void *x, int x_dtype, const float *R, void *y, int y_dtype, int64_t n, int d,
                         int inverse, float out_scale, hipStream_t s) {
  if (R == nullptr) {
    const int64_t m = n * d;
    const int grid = grid_for(m, 256, 4096);
    if (x_dtype == 0 && y_dtype == 0) scale_kernel<<<grid, 256, 0, s>>>((const float *)x, (float *)y, m, out_scale);
    else if (x_dtype == 0) scale_kernel<<<grid, 256, 0, s>>>((const float *)x, (half_t *)y, m, out_scale);
    else if (y_dtype == 0) scale_kernel<<<grid, 256, 0, s>>>((const half_t *)x, (float *)y, m, out_scale);
    else scale_kernel<<<grid, 256, 0, s>>>((const half_t *)x, (half_t *)y, m, out_scale);
    return hipGetLastError();
  }
  if (d == 128) {
    if (inverse) rotate_dispatch<128, true>(x, x_dtype, R, y, y_dtype, n, out_scale, s);
    else rotate_dispatch<128, false>(x, x_dtype, R, y, y_dtype, n, out_scale, s);
  } else {
    if (inverse) rotate_dispatch<64, true>(x, x_dtype, R, y, y_dtype, n, out_scale, s);
    else rotate_dispatch<64, false>(x, x_dtype, R, y, y_dtype, n, out_scale, s);
  }
  return hipGetLastError();
}

// The exact encoders keep a row of R in each thread's registers, loaded once
// per workgroup: one resident round of workgroups loops over the tiles (two
// per CU at d = 128, whose kernels take 2 waves per SIMD; three at d = 64).
static int exact_grid(int64_t n, int d) {
  return grid_for(n, kExactChains * (256 / d), (d == 128 ? 2 : 3) * device_compute_units());
}

hipError_t launch_encode_exact(const EncodeArgs &a, int x_dtype, hipStream_t s) {
  if (tiled_encode_ok(a, x_dtype)) return launch_encode_tiled(a, x_dtype, s);
  const int64_t n = a.n_outer * a.n_inner;
  const int grid = exact_grid(n, a.d);
#define PQKV_EE(DD, BB)                                                            \
  do {                                                                             \
    if (x_dtype == 0) encode_exact_kernel<DD, BB, float><<<grid, 256, 0, s>>>(a);  \
    else if (x_dtype == 1) encode_exact_kernel<DD, BB, half_t><<<grid, 256, 0, s>>>(a); \
    else encode_exact_kernel<DD, BB, bf16_t><<<grid, 256, 0, s>>>(a);              \
  } while (0)
  if (a.d == 128 && a.bits == 4) PQKV_EE(128, 4);
  else if (a.d == 128 && a.bits == 2) PQKV_EE(128, 2);
  else if (a.d == 64 && a.bits == 4) PQKV_EE(64, 4);
  else PQKV_EE(64, 2);
#undef PQKV_EE
  return hipGetLastError();
}

hipError_t launch_encode_soa(const float *x, const float *R, const float *codebook, int n_levels, float *radius,
                             uint8_t *packed, int64_t n, int d, hipStream_t s) {
  if (tiled_soa_ok(x, R, packed, n, d)) return launch_encode_soa_tiled(x, R, codebook, n_levels, radius, packed, n, d, s);
  const int grid = exact_grid(n, d);
  if (d == 128) encode_soa_kernel<128><<<grid, 256, 0, s>>>(x, R, codebook, n_levels, radius, packed, n);
  else encode_soa_kernel<64><<<grid, 256, 0, s>>>(x, R, codebook, n_levels, radius, packed, n);
  return hipGetLastError();
}

hipError_t launch_soa_to_blocks(const uint8_t *packed, const float *radius, uint8_t *blocks, int64_t n, int d,
                                hipStream_t s) {
  const int64_t total = n * (d / 2 + d / 32);
  soa_to_blocks_kernel<<<grid_for(total, 256), 256, 0, s>>>(packed, radius, blocks, n, d);
  return hipGetLastError();
}

hipError_t launch_blocks_to_soa(const uint8_t *blocks, uint8_t *packed, float *radius, int64_t n, int d,
                                hipStream_t s) {
  const int64_t total = n * (d / 2 + 1);
  blocks_to_soa_kernel<<<grid_for(total, 256), 256, 0, s>>>(blocks, packed, radius, n, d);
  return hipGetLastError();
}

}  // namespace pqkv
