// GGML_TYPE_PQ4: the block_pq4 format as a ggml type, and the two HIP
// backend ops a ggml backend needs to keep a KV cache in it.
//
// The reference's llama.cpp integration stores its cache as Q4_0 and never
// reaches its PolarQuant kernels from the graph (integration/polarquant-kv.patch:
// 1130-1137, 1303-1362, 1385-1404). Here the type is defined the way ggml
// defines a quantized type, over the format the kernels of this library read:
//   - blocks of PQKV_GGML_QK_PQ4 = 32 elements, PQKV_GGML_PQ4_TYPE_SIZE = 18
//     bytes ({fp16 radius; uint8 qs[16]}, README.md:73-78);
//   - a row holds whole heads of head_dim elements; each head is rotated by
//     the state's R (Gram-Schmidt over rand() after srand(42), patch:549-579),
//     its fp32 radius is the 128-slot tree of squares
//     (csrc/flash_turboquant.cu:141-148) stored as fp16 in each of its blocks,
//     and every coordinate of the direction gets the first nearest entry of
//     the 4-bit table of patch:978-983 (two codes per byte, low nibble first);
//   - the value of a head is (r16 * c[code]) R, rotated back.
// The CPU type traits (to_float / from_float_ref) use the FMA chains and the
// rounding of the GPU encoder, so a row quantised on the host and one copied
// on the device are the same bytes.
//
// Backend ops (device pointers, ggml's ne / nb conventions: ne[0] fastest,
// nb in bytes):
//   cpy            f32 / f16 rows -> PQ4 rows (the KV-cache store);
//   flash_attn_ext softmax(scale Q K^T + mask) V over PQ4 K and V views,
//                  output [d][Hq][n_q][n_seq] f32 (ggml's permuted result).
#include "../../include/pqkv.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <vector>

#include "pqkv_ggml_format.h"
#include "pqkv_launch.h"

namespace {

constexpr int kQK = PQKV_GGML_QK_PQ4;
constexpr int kBlockBytes = PQKV_GGML_PQ4_TYPE_SIZE;

// IEEE fp32 -> fp16 bits, round to nearest even (overflow to inf, NaN kept).
uint16_t f32_to_f16_bits(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);  // rounds past 65504
  if (ax < 0x38800000u) {
    // fp16 subnormal or zero: value = m * 2^-24, m = round(|f| * 2^24)
    if (ax < 0x33000000u) return (uint16_t)sign;  // below half the smallest subnormal
    const int e = (int)(ax >> 23);
    const uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u;
    const int shift = 126 - e;                    // 14 .. 24
    uint32_t m = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (m & 1u))) ++m;
    return (uint16_t)(sign | m);
  }
  uint32_t h = ((ax >> 13) - (112u << 10));
  const uint32_t rem = ax & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
  return (uint16_t)(sign | h);
}

float f16_bits_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1F, m = h & 0x3FFu;
  uint32_t x;
  if (e == 0) {
    if (m == 0) {
      x = sign;
    } else {
      float f = std::ldexp((float)m, -24);
      std::memcpy(&x, &f, 4);
      x |= sign;
    }
  } else if (e == 31) {
    x = sign | 0x7F800000u | (m << 13);
  } else {
    x = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  std::memcpy(&f, &x, 4);
  return f;
}

// One head of d (64 or 128) elements -> d / 32 blocks, with the GPU
// encoder's arithmetic: each rotated coordinate one fp32 FMA chain over k
// ascending, the squares and the tree additions rounded one at a time, the
// correctly rounded square root, IEEE division, the strict '<' scan, the
// radius stored as fp16 saturated at 65504.
void encode_head(const float *x, const float *R, const float *cb, int d, uint8_t *out) {
  float y[128], buf[128];
  for (int j = 0; j < d; ++j) {
    float acc = 0.0f;
    for (int k = 0; k < d; ++k) acc = std::fma(x[k], R[(size_t)j * d + k], acc);
    y[j] = acc;
  }
  for (int t = 0; t < 128; ++t) buf[t] = t < d ? y[t] * y[t] : 0.0f;  // built with -ffp-contract=off
  for (int s = 64; s > 0; s >>= 1)
    for (int t = 0; t < s; ++t) buf[t] = buf[t] + buf[t + s];
  const float r = (float)std::sqrt((double)buf[0]);
  const bool nz = r > 1e-30f;
  uint8_t codes[128];
  for (int j = 0; j < d; ++j) {
    const float dir = nz ? y[j] / r : 0.0f;
    int best = 0;
    float bd = 1e30f;
    for (int i = 0; i < 16; ++i) {
      const float e = std::fabs(dir - cb[i]);
      if (e < bd) {
        bd = e;
        best = i;
      }
    }
    codes[j] = (uint8_t)best;
  }
  const uint16_t r16 = f32_to_f16_bits(r > 65504.0f ? 65504.0f : r);
  for (int b = 0; b < d / kQK; ++b) {
    uint8_t *blk = out + (size_t)b * kBlockBytes;
    blk[0] = (uint8_t)(r16 & 0xFF);
    blk[1] = (uint8_t)(r16 >> 8);
    for (int i = 0; i < kQK / 2; ++i)
      blk[2 + i] = (uint8_t)(codes[kQK * b + 2 * i] | (codes[kQK * b + 2 * i + 1] << 4));
  }
}

// d / 32 blocks -> one head: r16 c[code], then y_j = sum_k v_k R[k][j] as one
// FMA chain over k ascending (the dequantise kernel's order).
void decode_head(const uint8_t *in, const float *R, const float *cb, int d, float *y) {
  float v[128];
  for (int b = 0; b < d / kQK; ++b) {
    const uint8_t *blk = in + (size_t)b * kBlockBytes;
    const float r = f16_bits_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
    for (int i = 0; i < kQK / 2; ++i) {
      v[kQK * b + 2 * i] = r * cb[blk[2 + i] & 15];
      v[kQK * b + 2 * i + 1] = r * cb[blk[2 + i] >> 4];
    }
  }
  for (int j = 0; j < d; ++j) {
    float acc = 0.0f;
    for (int k = 0; k < d; ++k) acc = std::fma(v[k], R[(size_t)k * d + j], acc);
    y[j] = acc;
  }
}

// The rotation of the default type (head_dim 64 or 128), generated once.
const float *default_rotation(int d) {
  static std::once_flag once[2];
  static std::vector<float> R[2];
  const int i = d == 128 ? 1 : 0;
  std::call_once(once[i], [&] {
    R[i].resize((size_t)d * d);
    pqkv::gram_schmidt_rotation(R[i].data(), d, 42);
  });
  return R[i].data();
}

bool heads_ok(int64_t k, int d) { return (d == 64 || d == 128) && k >= 0 && k % d == 0; }

}  // namespace

extern "C" {

int pqkv_pq4_quantize_rows_host(const float *x, void *y, int64_t k, int head_dim, const float *R,
                                const float *codebook) {
  if (!heads_ok(k, head_dim))
    return pqkv::fail_status(PQKV_ERR_INVALID, "pq4 rows: k=%lld is not whole heads of head_dim=%d (64 or 128)",
                             (long long)k, head_dim);
  if (k > 0 && (!x || !y || !R || !codebook)) return pqkv::fail_status(PQKV_ERR_INVALID, "pq4 rows: null pointer");
  const int64_t heads = k / head_dim;
  const int64_t hb = (int64_t)head_dim / kQK * kBlockBytes;
  for (int64_t h = 0; h < heads; ++h)
    encode_head(x + h * head_dim, R, codebook, head_dim, (uint8_t *)y + h * hb);
  return PQKV_OK;
}

int pqkv_pq4_dequantize_rows_host(const void *x, float *y, int64_t k, int head_dim, const float *R,
                                  const float *codebook) {
  if (!heads_ok(k, head_dim))
    return pqkv::fail_status(PQKV_ERR_INVALID, "pq4 rows: k=%lld is not whole heads of head_dim=%d (64 or 128)",
                             (long long)k, head_dim);
  if (k > 0 && (!x || !y || !R || !codebook)) return pqkv::fail_status(PQKV_ERR_INVALID, "pq4 rows: null pointer");
  const int64_t heads = k / head_dim;
  const int64_t hb = (int64_t)head_dim / kQK * kBlockBytes;
  for (int64_t h = 0; h < heads; ++h)
    decode_head((const uint8_t *)x + h * hb, R, codebook, head_dim, y + h * head_dim);
  return PQKV_OK;
}

int pqkv_ggml_pq4_rotation(float *R, int head_dim) {
  if (head_dim != 64 && head_dim != 128)
    return pqkv::fail_status(PQKV_ERR_UNSUPPORTED, "pq4 rotation: head_dim=%d (64 or 128)", head_dim);
  if (!R) return pqkv::fail_status(PQKV_ERR_INVALID, "pq4 rotation: null pointer");
  std::memcpy(R, default_rotation(head_dim), sizeof(float) * head_dim * head_dim);
  return PQKV_OK;
}

void pqkv_ggml_quantize_row_pq4_ref(const float *x, void *y, int64_t k) {
  if (pqkv_pq4_quantize_rows_host(x, y, k, 128, default_rotation(128), pqkv::kGgmlCodebook4) != PQKV_OK)
    fprintf(stderr, "PolarQuant (HIP): quantize_row_pq4: %s\n", pqkv_last_error());
}

void pqkv_ggml_dequantize_row_pq4(const void *x, float *y, int64_t k) {
  if (pqkv_pq4_dequantize_rows_host(x, y, k, 128, default_rotation(128), pqkv::kGgmlCodebook4) != PQKV_OK)
    fprintf(stderr, "PolarQuant (HIP): dequantize_row_pq4: %s\n", pqkv_last_error());
}

int pqkv_ggml_cpy_pq4(const polarquant_state *st, const void *src, int src_type, const int64_t ne[4],
                      const size_t nb[4], void *dst, const size_t nb_dst[4], void *stream) {
  if (!st || !st->rotation || !st->codebook || st->n_bits != 4)
    return pqkv::fail_status(PQKV_ERR_INVALID, "ggml cpy: a 4-bit polarquant state is required");
  if (!ne || !nb || !nb_dst) return pqkv::fail_status(PQKV_ERR_INVALID, "ggml cpy: null shape");
  const int d = st->head_dim;
  if (src_type != PQKV_F32 && src_type != PQKV_F16)
    return pqkv::fail_status(PQKV_ERR_UNSUPPORTED, "ggml cpy: source type %d (f32 or f16)", src_type);
  for (int i = 0; i < 4; ++i)
    if (ne[i] < 0) return pqkv::fail_status(PQKV_ERR_INVALID, "ggml cpy: ne[%d]=%lld", i, (long long)ne[i]);
  if (ne[0] % d) return pqkv::fail_status(PQKV_ERR_INVALID, "ggml cpy: ne[0]=%lld is not whole heads of %d",
                                          (long long)ne[0], d);
  const size_t es = src_type == PQKV_F32 ? 4 : 2;
  if (nb[0] != es || nb[1] % es || nb[2] % es || nb[3] % es)
    return pqkv::fail_status(PQKV_ERR_UNSUPPORTED, "ggml cpy: source rows must be contiguous and element-aligned");
  if (nb_dst[0] != (size_t)kBlockBytes || nb_dst[1] % 2 || nb_dst[2] % 2 || nb_dst[3] % 2 || (uintptr_t)dst % 2)
    return pqkv::fail_status(PQKV_ERR_UNSUPPORTED, "ggml cpy: destination rows must be contiguous blocks, 2-byte aligned");
  if ((uintptr_t)src % es) return pqkv::fail_status(PQKV_ERR_INVALID, "ggml cpy: misaligned source");
  const int64_t n = ne[0] * ne[1] * ne[2] * ne[3];
  if (n == 0) return PQKV_OK;
  if (!src || !dst) return pqkv::fail_status(PQKV_ERR_INVALID, "ggml cpy: null pointer");
  pqkv::EncodeArgs a;
  std::memset(&a, 0, sizeof(a));
  a.R = st->rotation;
  a.codebook = st->codebook;
  a.bits = 4;
  a.d = d;
  a.x_outer_stride = (int64_t)(nb[1] / es);
  a.blocks_outer_stride = (int64_t)nb_dst[1];
  a.n_outer = ne[1];
  a.n_inner = ne[0] / d;
  for (int64_t i3 = 0; i3 < ne[3]; ++i3)
    for (int64_t i2 = 0; i2 < ne[2]; ++i2) {
      a.x = (const uint8_t *)src + i2 * nb[2] + i3 * nb[3];
      a.blocks = (uint8_t *)dst + i2 * nb_dst[2] + i3 * nb_dst[3];
      const hipError_t e = pqkv::launch_encode_exact(a, src_type, (hipStream_t)stream);
      if (e != hipSuccess) return pqkv::report_hip_error(e, "ggml cpy launch");
    }
  return PQKV_OK;
}

}  // extern "C"

namespace {

// The validated shape of one flash_attn_ext call.
struct FaShape {
  int d, n_q, Hq, n_seq, n_kv, Hkv;
  int splits, tps;
  size_t q_off, part_off, bytes;
};

int fa_shape(const polarquant_state *st, const int64_t ne_q[4], const int64_t ne_k[4], FaShape *f) {
  if (!st || !st->rotation || !st->codebook || st->n_bits != 4)
    return pqkv::fail_status(PQKV_ERR_INVALID, "ggml flash_attn_ext: a 4-bit polarquant state is required");
  if (!ne_q || !ne_k) return pqkv::fail_status(PQKV_ERR_INVALID, "ggml flash_attn_ext: null shape");
  const int d = st->head_dim;
  if (ne_q[0] != d || ne_k[0] != d)
    return pqkv::fail_status(PQKV_ERR_INVALID, "ggml flash_attn_ext: head sizes q %lld, k %lld, state %d",
                             (long long)ne_q[0], (long long)ne_k[0], d);
  for (int i = 1; i < 4; ++i)
    if (ne_q[i] < 0 || ne_q[i] > INT32_MAX || ne_k[i] < 0 || ne_k[i] > INT32_MAX)
      return pqkv::fail_status(PQKV_ERR_INVALID, "ggml flash_attn_ext: ne[%d] out of range", i);
  f->d = d;
  f->n_q = (int)ne_q[1];
  f->Hq = (int)ne_q[2];
  f->n_seq = (int)ne_q[3];
  f->n_kv = (int)ne_k[1];
  f->Hkv = (int)ne_k[2];
  if (f->Hkv <= 0 || f->Hq % f->Hkv)
    return pqkv::fail_status(PQKV_ERR_INVALID, "ggml flash_attn_ext: %d query heads over %d kv heads", f->Hq, f->Hkv);
  if (ne_k[3] != 1 && ne_k[3] != ne_q[3])
    return pqkv::fail_status(PQKV_ERR_INVALID, "ggml flash_attn_ext: %lld kv sequences for %lld query sequences",
                             (long long)ne_k[3], (long long)ne_q[3]);
  const int64_t rows = (int64_t)f->n_seq * f->n_q;
  // one workgroup row per (query row, kv head): the grid's second dimension
  if (rows * f->Hkv > 65535 || rows * f->Hq > INT32_MAX)
    return pqkv::fail_status(PQKV_ERR_UNSUPPORTED, "ggml flash_attn_ext: %lld query rows x %d kv heads exceed 65535",
                             (long long)rows, f->Hkv);
  f->splits = 1;
  f->tps = 0;
  // (a workgroup row per four kv heads when the kernel takes one per wave)
  const int64_t wg_rows = pqkv::ggml_heads_per_wave(f->Hkv) ? rows * f->Hkv / 4 : rows * f->Hkv;
  if (rows > 0 && f->n_kv > 0) pqkv::mfma_split_plan(wg_rows, f->n_kv, &f->splits, &f->tps);
  size_t pq_off;
  f->bytes = pqkv::decode_workspace_layout((int)rows, f->Hq, f->splits, d, &f->q_off, &f->part_off, &pq_off);
  return PQKV_OK;
}

}  // namespace

extern "C" {

size_t pqkv_ggml_flash_attn_ext_pq4_workspace_bytes(const polarquant_state *st, const int64_t ne_q[4],
                                                    const int64_t ne_k[4]) {
  FaShape f;
  return fa_shape(st, ne_q, ne_k, &f) == PQKV_OK ? f.bytes : 0;
}

int pqkv_ggml_flash_attn_ext_pq4(const polarquant_state *st, const float *q, const int64_t ne_q[4],
                                 const size_t nb_q[4], const void *k, const int64_t ne_k[4], const size_t nb_k[4],
                                 const void *v, const int64_t ne_v[4], const size_t nb_v[4], const void *mask,
                                 const int64_t ne_m[4], const size_t nb_m[4], float scale, float max_bias,
                                 float logit_softcap, float *dst, void *workspace, size_t workspace_bytes,
                                 void *stream) {
  FaShape f;
  const int rc = fa_shape(st, ne_q, ne_k, &f);
  if (rc != PQKV_OK) return rc;
  if (!nb_q || !nb_k || !ne_v || !nb_v) return pqkv::fail_status(PQKV_ERR_INVALID, "ggml flash_attn_ext: null shape");
  for (int i = 0; i < 4; ++i)
    if (ne_v[i] != ne_k[i])
      return pqkv::fail_status(PQKV_ERR_INVALID, "ggml flash_attn_ext: v ne[%d]=%lld differs from k's %lld", i,
                               (long long)ne_v[i], (long long)ne_k[i]);
  if (max_bias != 0.0f || logit_softcap != 0.0f)
    return pqkv::fail_status(PQKV_ERR_UNSUPPORTED, "ggml flash_attn_ext: max_bias and logit_softcap must be 0");
  if (!std::isfinite(scale)) return pqkv::fail_status(PQKV_ERR_INVALID, "ggml flash_attn_ext: scale not finite");
  if (nb_q[0] != 4 || nb_q[1] % 4 || nb_q[2] % 4 || nb_q[3] % 4 || (uintptr_t)q % 4)
    return pqkv::fail_status(PQKV_ERR_UNSUPPORTED, "ggml flash_attn_ext: q must be f32 with contiguous rows");
  for (const size_t *nb : {nb_k, nb_v})
    if (nb[0] != (size_t)kBlockBytes || nb[1] % 2 || nb[2] % 2 || nb[3] % 2)
      return pqkv::fail_status(PQKV_ERR_UNSUPPORTED, "ggml flash_attn_ext: k / v must be PQ4 rows, 2-byte strides");
  if ((uintptr_t)k % 2 || (uintptr_t)v % 2 || (uintptr_t)dst % 4)
    return pqkv::fail_status(PQKV_ERR_INVALID, "ggml flash_attn_ext: misaligned k, v or dst");
  // the kernel addresses a stream with 32-bit byte offsets
  if ((int64_t)f.n_kv * (int64_t)std::max(nb_k[1], nb_v[1]) >= ((int64_t)1 << 31))
    return pqkv::fail_status(PQKV_ERR_UNSUPPORTED, "ggml flash_attn_ext: n_kv * token stride must stay below 2^31");
  const uint16_t *mrow = (const uint16_t *)mask;
  int64_t m_row = 0, m_seq = 0;
  if (mask) {
    if (!ne_m || !nb_m) return pqkv::fail_status(PQKV_ERR_INVALID, "ggml flash_attn_ext: null mask shape");
    if (ne_m[0] < f.n_kv || ne_m[1] < f.n_q || ne_m[2] != 1 || (ne_m[3] != 1 && ne_m[3] != f.n_seq))
      return pqkv::fail_status(PQKV_ERR_INVALID, "ggml flash_attn_ext: mask [%lld, %lld, %lld, %lld] for n_kv=%d n_q=%d",
                               (long long)ne_m[0], (long long)ne_m[1], (long long)ne_m[2], (long long)ne_m[3],
                               f.n_kv, f.n_q);
    if (nb_m[0] != 2 || nb_m[1] % 2 || nb_m[3] % 2 || (uintptr_t)mask % 2)
      return pqkv::fail_status(PQKV_ERR_UNSUPPORTED, "ggml flash_attn_ext: the mask must be f16 with contiguous rows");
    m_row = (int64_t)(nb_m[1] / 2);
    m_seq = ne_m[3] == 1 ? 0 : (int64_t)(nb_m[3] / 2);
  }
  const int64_t rows = (int64_t)f.n_seq * f.n_q;
  if (rows == 0 || f.Hq == 0) return PQKV_OK;
  if (!q || !dst) return pqkv::fail_status(PQKV_ERR_INVALID, "ggml flash_attn_ext: null pointer");
  hipStream_t s = (hipStream_t)stream;
  if (f.n_kv == 0)
    return pqkv::report_hip_error(pqkv::launch_fill_zero(dst, (size_t)rows * f.Hq * f.d * 4, s),
                                  "ggml flash_attn_ext zero fill");
  if (!k || !v) return pqkv::fail_status(PQKV_ERR_INVALID, "ggml flash_attn_ext: null k or v");
  if (!workspace || workspace_bytes < f.bytes)
    return pqkv::fail_status(PQKV_ERR_WORKSPACE, "ggml flash_attn_ext: workspace %zu < %zu bytes", workspace_bytes,
                             f.bytes);
  float *q32 = (float *)((char *)workspace + f.q_off);
  float *part = (float *)((char *)workspace + f.part_off);
  const float kLog2e = 1.4426950408889634f;
  int tok = pqkv::prof_begin("ggml_fa_rotate", s);
  hipError_t e = pqkv::launch_rotate_rows(q, (int64_t)(nb_q[1] / 4), (int64_t)(nb_q[2] / 4), (int64_t)(nb_q[3] / 4),
                                          f.n_q, f.Hq, f.n_seq, st->rotation, q32, f.d, scale * kLog2e, s);
  pqkv::prof_end(tok, s);
  if (e != hipSuccess) return pqkv::report_hip_error(e, "ggml flash_attn_ext query rotation");

  pqkv::DecodeArgs a;
  std::memset(&a, 0, sizeof(a));
  a.q = q32;
  a.k_cache = (const uint8_t *)k;
  a.v_cache = (const uint8_t *)v;
  a.k_cb = a.v_cb = st->codebook;
  a.cb_levels = 16;
  a.part = part;
  a.B = (int)rows;
  a.Hq = f.Hq;
  a.Hkv = f.Hkv;
  a.gq = f.Hq / f.Hkv;
  a.S = f.n_kv;
  a.S_max = f.n_kv;
  a.d = f.d;
  a.splits = f.splits;
  a.tokens_per_split = f.tps;
  a.split_base = 0;
  a.split_stride = f.splits;
  a.n_heads = f.Hkv;
  a.listed = 0;
  a.k_tok_stride = (int64_t)nb_k[1];
  a.v_tok_stride = (int64_t)nb_v[1];
  a.k_head_stride = (int64_t)nb_k[2];
  a.v_head_stride = (int64_t)nb_v[2];
  a.k_batch_stride = ne_k[3] == 1 ? 0 : (int64_t)nb_k[3];
  a.v_batch_stride = ne_v[3] == 1 ? 0 : (int64_t)nb_v[3];
  a.rows_per_seq = f.n_q;
  a.mask = mrow;
  a.mask_row_stride = m_row;
  a.mask_seq_stride = m_seq;
  // query heads of a kv head in launches of at most kMaxGroup
  const int n_sub = (a.gq + pqkv::kMaxGroup - 1) / pqkv::kMaxGroup;
  int off = 0;
  for (int i = 0; i < n_sub; ++i) {
    a.q_off = off;
    a.g = a.gq / n_sub + (i < a.gq % n_sub ? 1 : 0);
    tok = pqkv::prof_begin("ggml_fa_split", s, true);
    e = hipSuccess;
    for (int rep = 0, nrep = pqkv::prof_repeats(); rep < nrep && e == hipSuccess; ++rep)
      e = pqkv::launch_decode_mfma_ggml(a, s);
    pqkv::prof_end(tok, s);
    if (e != hipSuccess) return pqkv::report_hip_error(e, "ggml flash_attn_ext split launch");
    off += a.g;
  }
  tok = pqkv::prof_begin("ggml_fa_merge", s, true);
  e = hipSuccess;
  for (int rep = 0, nrep = pqkv::prof_repeats(); rep < nrep && e == hipSuccess; ++rep)
    e = pqkv::launch_decode_merge(part, st->rotation, dst, PQKV_F32, (int)(rows * f.Hq), f.splits, f.d, s);
  pqkv::prof_end(tok, s);
  return pqkv::report_hip_error(e, "ggml flash_attn_ext merge launch");
}

}  // extern "C"
