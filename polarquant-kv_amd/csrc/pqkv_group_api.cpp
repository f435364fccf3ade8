// C ABI of the reference's GPU group format (CompressedKVCacheGPU,
// src/polarquant_kv_cuda/types.py:7-21): compress_gpu, decompress_gpu, the
// QJL sketch of compute_signatures_gpu and attention on the format
// (compressed_attention_gpu; the fused kernels of csrc/polarquant_full.cu),
// plus the reference's polarquant_full pybind surface. Every argument is
// checked here, in host code, before any HIP call.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>

#include "../../include/pqkv.h"
#include "pqkv_launch.h"

namespace {

constexpr int kMaxD = 256;

int fail(int code, const char *fmt, int a = 0, int b = 0, int c = 0) {
  return pqkv::fail_status(code, fmt, a, b, c);
}
int hip_status(hipError_t e, const char *what) { return pqkv::report_hip_error(e, what); }
bool param_dtype_ok(int t) { return t == PQKV_F32 || t == PQKV_F16; }
bool in_dtype_ok(int t) { return t == PQKV_F32 || t == PQKV_F16 || t == PQKV_BF16; }
int store_bits(int bits) { return bits == 4 ? 4 : bits == 2 ? 2 : 8; }

// Fused attention's layout needs: every unit of 8 codes (and every code
// dword) inside one group, d_pad <= 256.
int attn_shape_check(int d, int gs, int bits) {
  if (d < 1 || d > kMaxD) return fail(PQKV_ERR_UNSUPPORTED, "group_attn: d=%d (1..256)", d);
  if (gs < 1 || gs > d) return fail(PQKV_ERR_INVALID, "group_attn: group_size=%d (1..d=%d)", gs, d);
  const int ng = (d + gs - 1) / gs, dpad = ng * gs;
  const int unit = store_bits(bits) == 2 ? 16 : 8;
  if (gs % unit || dpad > kMaxD)
    return pqkv::fail_status(PQKV_ERR_UNSUPPORTED,
                             "group_attn: group_size=%d must be a multiple of %d for %d-bit codes and d_pad=%d at "
                             "most 256", gs, unit, bits, dpad);
  return PQKV_OK;
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Workspace: rotated query rows [rows][dpad], P q rows [rows][m], split
// partials [rows][splits][d + 2].
size_t attn_layout(int64_t rows, int dpad, int m, int splits, int d, size_t *pq_off, size_t *part_off) {
  size_t off = align256((size_t)rows * dpad * 4);
  if (pq_off) *pq_off = off;
  off += align256((size_t)rows * (m > 0 ? m : 0) * 4);
  if (part_off) *part_off = off;
  off += align256((size_t)rows * splits * (d + 2) * 4);
  return off;
}

// VALU kernel: about four workgroups per compute unit
int attn_target() { return 4 * pqkv::device_compute_units(); }
constexpr int kAttnPlanMaxTarget = 2048;

}  // namespace

extern "C" {

int pqkv_group_gpu_compress(const void *x, int x_dtype, const float *R, const float *Rt, int64_t n, int d, int n_bits,
                            int group_size, void *radius, uint8_t *codes, void *mins, void *scales, int param_dtype,
                            float *residual, void *stream) {
  if (n < 0) return fail(PQKV_ERR_INVALID, "group_gpu_compress: n < 0");
  if (d < 1 || d > kMaxD) return fail(PQKV_ERR_UNSUPPORTED, "group_gpu_compress: d=%d (1..256)", d);
  if (n_bits < 2 || n_bits > 8) return fail(PQKV_ERR_INVALID, "group_gpu_compress: n_bits=%d (2..8)", n_bits);
  if (group_size < 1 || group_size > d)
    return fail(PQKV_ERR_INVALID, "group_gpu_compress: group_size=%d (1..d=%d)", group_size, d);
  const int dpad = (d + group_size - 1) / group_size * group_size;
  if ((n_bits == 4 && dpad % 2) || (n_bits == 2 && dpad % 4))
    return fail(PQKV_ERR_INVALID, "group_gpu_compress: d_pad=%d does not pack %d-bit codes", dpad, n_bits);
  if (!in_dtype_ok(x_dtype) || !param_dtype_ok(param_dtype))
    return fail(PQKV_ERR_UNSUPPORTED, "group_gpu_compress: dtype x=%d params=%d", x_dtype, param_dtype);
  if (n == 0) return PQKV_OK;
  if (!x || !Rt || !radius || !codes || !mins || !scales || (residual && !R))
    return fail(PQKV_ERR_INVALID, "group_gpu_compress: null pointer");
  return hip_status(pqkv::launch_group_gpu_compress(x, x_dtype, Rt, R, n, d, n_bits, group_size, radius, codes, mins,
                                                    scales, param_dtype, residual, (hipStream_t)stream),
                    "group_gpu_compress launch");
}

int pqkv_group_gpu_decompress(const void *radius, const uint8_t *codes, const void *mins, const void *scales,
                              int param_dtype, const float *R, int64_t n, int d, int n_bits, int group_size, void *out,
                              int out_dtype, void *stream) {
  if (n < 0) return fail(PQKV_ERR_INVALID, "group_gpu_decompress: n < 0");
  if (d < 1 || d > kMaxD) return fail(PQKV_ERR_UNSUPPORTED, "group_gpu_decompress: d=%d (1..256)", d);
  if (n_bits < 2 || n_bits > 8) return fail(PQKV_ERR_INVALID, "group_gpu_decompress: n_bits=%d (2..8)", n_bits);
  if (group_size < 1 || group_size > d)
    return fail(PQKV_ERR_INVALID, "group_gpu_decompress: group_size=%d (1..d=%d)", group_size, d);
  if (!param_dtype_ok(param_dtype) || !param_dtype_ok(out_dtype))
    return fail(PQKV_ERR_UNSUPPORTED, "group_gpu_decompress: dtype params=%d out=%d", param_dtype, out_dtype);
  if (n == 0) return PQKV_OK;
  if (!radius || !codes || !mins || !scales || !R || !out)
    return fail(PQKV_ERR_INVALID, "group_gpu_decompress: null pointer");
  return hip_status(pqkv::launch_group_gpu_decompress(radius, codes, mins, scales, param_dtype, R, n, d, n_bits,
                                                      group_size, out, out_dtype, (hipStream_t)stream),
                    "group_gpu_decompress launch");
}

int pqkv_qjl_sketch(const void *x, int x_dtype, const float *x_hat, const double *Pt, int64_t n, int d, int m,
                    uint8_t *signs, void *norms, int norm_dtype, void *stream) {
  if (n < 0 || m < 1 || m > 4096) return fail(PQKV_ERR_INVALID, "qjl_sketch: n < 0 or m=%d (1..4096)", m);
  if (d < 1 || d > kMaxD) return fail(PQKV_ERR_UNSUPPORTED, "qjl_sketch: d=%d (1..256)", d);
  if (!in_dtype_ok(x_dtype) || !param_dtype_ok(norm_dtype))
    return fail(PQKV_ERR_UNSUPPORTED, "qjl_sketch: dtype x=%d norms=%d", x_dtype, norm_dtype);
  if (n == 0) return PQKV_OK;
  if (!x || !Pt || !signs || !norms) return fail(PQKV_ERR_INVALID, "qjl_sketch: null pointer");
  return hip_status(pqkv::launch_qjl_sketch(x, x_dtype, x_hat, Pt, n, d, m, signs, norms, norm_dtype,
                                            (hipStream_t)stream),
                    "qjl_sketch launch");
}

size_t pqkv_group_attn_workspace_bytes(int B, int Hq, int Hkv, int S, int d, int group_size, int m) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || S < 0 || d < 1 || d > kMaxD || group_size < 1 || group_size > d || m < 0)
    return 0;
  const int dpad = (d + group_size - 1) / group_size * group_size;
  int splits = 1, tps = 0;
  pqkv::decode_plan_for((int64_t)B * Hkv, S > 0 ? S : 1, kAttnPlanMaxTarget, &splits, &tps);
  return attn_layout((int64_t)B * Hq, dpad, m, splits, d, nullptr, nullptr);
}

int pqkv_group_attn(const void *q, int q_dtype, const float *R, const float *P, int m, const uint8_t *k_codes,
                    const void *k_radius, const void *k_mins, const void *k_scales, const uint8_t *v_codes,
                    const void *v_radius, const void *v_mins, const void *v_scales, const uint8_t *qjl_signs,
                    const void *residual_norms, int n_bits, int param_dtype, int B, int Hq, int Hkv, int S, int S_max,
                    int d, int group_size, float scale, void *out, int out_dtype, void *workspace,
                    size_t workspace_bytes, void *stream) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || S < 0 || S_max < S)
    return fail(PQKV_ERR_INVALID, "group_attn: B=%d Hq=%d Hkv=%d", B, Hq, Hkv);
  if (Hq % Hkv) return fail(PQKV_ERR_INVALID, "group_attn: Hq=%d not a multiple of Hkv=%d", Hq, Hkv);
  if (n_bits < 2 || n_bits > 8) return fail(PQKV_ERR_INVALID, "group_attn: n_bits=%d (2..8)", n_bits);
  const int sc = attn_shape_check(d, group_size, n_bits);
  if (sc != PQKV_OK) return sc;
  if (!in_dtype_ok(q_dtype) || !param_dtype_ok(param_dtype) || !param_dtype_ok(out_dtype))
    return fail(PQKV_ERR_UNSUPPORTED, "group_attn: dtype q=%d params=%d out=%d", q_dtype, param_dtype, out_dtype);
  if ((qjl_signs == nullptr) != (P == nullptr)) return fail(PQKV_ERR_INVALID, "group_attn: qjl and P go together");
  if (qjl_signs && (m < 32 || m % 32 || m > 256))
    return fail(PQKV_ERR_UNSUPPORTED, "group_attn: QJL needs m a multiple of 32 up to 256, got %d", m);
  if (!(scale > 0.0f) || !std::isfinite(scale)) return fail(PQKV_ERR_INVALID, "group_attn: scale must be > 0");
  if (!q || !out) return fail(PQKV_ERR_INVALID, "group_attn: null query or output");
  if (S > 0 && (!k_codes || !k_radius || !k_mins || !k_scales || !v_codes || !v_radius || !v_mins || !v_scales))
    return fail(PQKV_ERR_INVALID, "group_attn: null cache field");
  const int dpad = (d + group_size - 1) / group_size * group_size;
  const int mm = qjl_signs ? m : 0;
  int splits = 1, tps = 0;
  pqkv::decode_plan_for((int64_t)B * Hkv, S > 0 ? S : 1, attn_target(), &splits, &tps);
  size_t pq_off = 0, part_off = 0;
  const size_t need = attn_layout((int64_t)B * Hq, dpad, mm, splits, d, &pq_off, &part_off);
  hipStream_t st = (hipStream_t)stream;
  if (S == 0) {
    const size_t ob = (size_t)B * Hq * d * (out_dtype == PQKV_F32 ? 4 : 2);
    return hip_status(pqkv::launch_fill_zero(out, ob, st), "group_attn zero fill");
  }
  if (!workspace || workspace_bytes < need)
    return pqkv::fail_status(PQKV_ERR_WORKSPACE, "group_attn: workspace %zu < %zu bytes", workspace_bytes, need);
  float *q_rot = (float *)workspace;
  float *pq = (float *)((char *)workspace + pq_off);
  float *part = (float *)((char *)workspace + part_off);
  const float kLog2e = 1.4426950408889634f;
  const int64_t rows = (int64_t)B * Hq;
  hipError_t e = pqkv::launch_group_qprep(q, q_dtype, R, qjl_signs ? P : nullptr, rows, d, dpad, mm, scale * kLog2e,
                                          q_rot, pq, st);
  if (e != hipSuccess) return hip_status(e, "group_attn query preparation");
  pqkv::GroupAttnArgsHost a;
  memset(&a, 0, sizeof(a));
  a.q = q_rot;
  a.pq = qjl_signs ? pq : nullptr;
  a.k_codes = k_codes;
  a.v_codes = v_codes;
  a.k_rad = k_radius;
  a.v_rad = v_radius;
  a.k_lo = k_mins;
  a.k_sc = k_scales;
  a.v_lo = v_mins;
  a.v_sc = v_scales;
  a.qjl = qjl_signs;
  a.res_norm = qjl_signs ? residual_norms : nullptr;
  a.part = part;
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.S = S;
  a.S_max = S_max;
  a.d = d;
  a.dpad = dpad;
  a.gs = group_size;
  a.bits = n_bits;
  a.pdt = param_dtype;
  a.m = mm;
  a.splits = splits;
  a.tps = tps;
  int tok = pqkv::prof_begin("group_attn_split", st, true);
  for (int rep = 0, nrep = pqkv::prof_repeats(); rep < nrep && e == hipSuccess; ++rep) e = pqkv::launch_group_attn(a, st);
  pqkv::prof_end(tok, st);
  if (e != hipSuccess) return hip_status(e, "group_attn split launch");
  tok = pqkv::prof_begin("group_attn_merge", st, true);
  for (int rep = 0, nrep = pqkv::prof_repeats(); rep < nrep && e == hipSuccess; ++rep)
    e = pqkv::launch_group_merge(part, R, out, out_dtype, rows, splits, d, st);
  pqkv::prof_end(tok, st);
  return hip_status(e, "group_attn merge launch");
}

// Codebook-format attention on the reference kernels' SoA cache at any head
// dim with d % 8 == 0, d <= 256 (the compat entry points' path for head dims
// the matrix-core kernels are not built for): q already rotated, output
// rotated, fp32 radii, 4-bit packed codes, a table of `levels` entries.
int pqkv_soa_attn_generic(const float *q_rot, const uint8_t *k_codes, const float *k_radius, const uint8_t *v_codes,
                          const float *v_radius, const float *codebook, int levels, int Hq, int Hkv, int S, int d,
                          float scale, float *out, void *workspace, size_t workspace_bytes, void *stream) {
  if (Hq <= 0 || Hkv <= 0 || Hq % Hkv || S < 0) return fail(PQKV_ERR_INVALID, "soa_attn: Hq=%d Hkv=%d S=%d", Hq, Hkv, S);
  if (d < 8 || d > kMaxD || d % 8) return fail(PQKV_ERR_UNSUPPORTED, "soa_attn: d=%d (a multiple of 8 up to 256)", d);
  if (levels < 1 || levels > 16) return fail(PQKV_ERR_UNSUPPORTED, "soa_attn: levels=%d (1..16)", levels);
  if (!(scale > 0.0f) || !std::isfinite(scale)) return fail(PQKV_ERR_INVALID, "soa_attn: scale must be > 0");
  if (!q_rot || !out || (S > 0 && (!k_codes || !k_radius || !v_codes || !v_radius || !codebook)))
    return fail(PQKV_ERR_INVALID, "soa_attn: null pointer");
  int splits = 1, tps = 0;
  pqkv::decode_plan_for(Hkv, S > 0 ? S : 1, attn_target(), &splits, &tps);
  size_t pq_off = 0, part_off = 0;
  const size_t need = attn_layout(Hq, d, 0, splits, d, &pq_off, &part_off);
  hipStream_t st = (hipStream_t)stream;
  if (S == 0) return hip_status(pqkv::launch_fill_zero(out, (size_t)Hq * d * 4, st), "soa_attn zero fill");
  if (!workspace || workspace_bytes < need)
    return pqkv::fail_status(PQKV_ERR_WORKSPACE, "soa_attn: workspace %zu < %zu bytes", workspace_bytes, need);
  float *qw = (float *)workspace;
  float *part = (float *)((char *)workspace + part_off);
  const float kLog2e = 1.4426950408889634f;
  hipError_t e = pqkv::launch_group_qprep(q_rot, PQKV_F32, nullptr, nullptr, Hq, d, d, 0, scale * kLog2e, qw, nullptr,
                                          st);
  if (e != hipSuccess) return hip_status(e, "soa_attn query scaling");
  pqkv::GroupAttnArgsHost a;
  memset(&a, 0, sizeof(a));
  a.q = qw;
  a.k_codes = k_codes;
  a.v_codes = v_codes;
  a.k_rad = k_radius;
  a.v_rad = v_radius;
  a.cb = codebook;
  a.cb_levels = levels;
  a.part = part;
  a.B = 1;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.S = S;
  a.S_max = S;
  a.d = d;
  a.dpad = d;
  a.gs = d;
  a.bits = 4;
  a.pdt = PQKV_F32;
  a.splits = splits;
  a.tps = tps;
  e = pqkv::launch_group_attn(a, st);
  if (e != hipSuccess) return hip_status(e, "soa_attn split launch");
  return hip_status(pqkv::launch_group_merge(part, nullptr, out, PQKV_F32, Hq, splits, d, st), "soa_attn merge");
}

size_t pqkv_soa_attn_generic_workspace_bytes(int Hq, int Hkv, int S, int d) {
  if (Hq <= 0 || Hkv <= 0 || S < 0 || d < 1 || d > kMaxD) return 0;
  int splits = 1, tps = 0;
  pqkv::decode_plan_for(Hkv, S > 0 ? S : 1, kAttnPlanMaxTarget, &splits, &tps);
  return attn_layout(Hq, d, 0, splits, d, nullptr, nullptr);
}

// ---- the reference's polarquant_full pybind surface (csrc/polarquant_full.cu:142-186) ----
// q [total_heads][D] fp32 in the original space; 4-bit codes [total_kv][S][D/2]
// (coordinate 2i low nibble), fp32 group minima and scales [total_kv][S][ng]
// and radii [total_kv][S]; out [total_heads][D] fp32 in the original space.
// q_rot, score and attn_out are the caller's fp32 scratch ([H][D], [H][S],
// [H][D]): score holds this call's workspace when it is large enough,
// otherwise a stream-ordered allocation is made and released.
void full_compressed_attention(int64_t q_ptr, int64_t R_ptr, int64_t pk_ptr, int64_t km_ptr, int64_t ks_ptr,
                               int64_t kr_ptr, int64_t pv_ptr, int64_t vm_ptr, int64_t vs_ptr, int64_t vr_ptr,
                               int64_t out_ptr, int64_t q_rot_ptr, int64_t score_ptr, int64_t attn_out_ptr,
                               int total_heads, int total_kv, int S, int D, int group_size, int num_groups,
                               float scale) {
  (void)q_rot_ptr;
  (void)attn_out_ptr;
  if (total_heads <= 0 || S <= 0 || D <= 0) return;
  if (total_kv <= 0 || total_heads % total_kv || group_size <= 0 || num_groups != (D + group_size - 1) / group_size) {
    fprintf(stderr, "PolarQuant (HIP): full_compressed_attention: unsupported heads=%d kv=%d D=%d gs=%d ng=%d\n",
            total_heads, total_kv, D, group_size, num_groups);
    return;
  }
  auto run = [&](void *ws, size_t bytes) {
    return pqkv_group_attn((const void *)q_ptr, PQKV_F32, (const float *)R_ptr, nullptr, 0, (const uint8_t *)pk_ptr,
                           (const void *)kr_ptr, (const void *)km_ptr, (const void *)ks_ptr, (const uint8_t *)pv_ptr,
                           (const void *)vr_ptr, (const void *)vm_ptr, (const void *)vs_ptr, nullptr, nullptr, 4,
                           PQKV_F32, 1, total_heads, total_kv, S, S, D, group_size, scale, (void *)out_ptr, PQKV_F32,
                           ws, bytes, nullptr);
  };
  int rc = PQKV_ERR_WORKSPACE;
  void *score = (void *)score_ptr;
  if (score && (uintptr_t)score % 256 == 0) rc = run(score, (size_t)total_heads * S * sizeof(float));
  if (rc == PQKV_ERR_WORKSPACE) {
    const size_t ws = pqkv_group_attn_workspace_bytes(1, total_heads, total_kv, S, D, group_size, 0);
    void *work = nullptr;
    if (hipMallocAsync(&work, ws, nullptr) != hipSuccess) {
      fprintf(stderr, "PolarQuant (HIP): full_compressed_attention: hipMallocAsync failed\n");
      return;
    }
    rc = run(work, ws);
    (void)hipFreeAsync(work, nullptr);
  }
  if (rc != PQKV_OK) fprintf(stderr, "PolarQuant (HIP): full_compressed_attention: %s\n", pqkv_last_error());
}

}  // extern "C"
