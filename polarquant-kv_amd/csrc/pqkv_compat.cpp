// Reference-compatible exports: the extern "C" surface of the reference's
// ggml CUDA backend (integration/polarquant-kv.patch:695-763), which
// llama.cpp binds with dlsym (patch:1508-1557). Same names, arguments, return
// types and ownership; SoA cache layout (packed u8 [N][D/2] + fp32 radius).
// Kernels are the library's own: the SoA encoder reproduces the reference's
// arithmetic exactly; attention runs the split-K matrix-core decode kernel
// reading the SoA codes and fp32 radii in place, with no rotation of the
// query or the output (these entry points take an already-rotated query and
// return a rotated output).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../../include/pqkv.h"
#include "pqkv_ggml_format.h"
#include "pqkv_launch.h"

namespace {

bool report(hipError_t e, const char *what) {
  if (e == hipSuccess) return true;
  fprintf(stderr, "PolarQuant (HIP): %s: %s\n", what, hipGetErrorString(e));
  return false;
}

}  // namespace

extern "C" {

polarquant_state *polarquant_init_c(int head_dim, int n_kv_heads, int n_q_heads, int n_layers, int n_kv_max,
                                    int n_bits) {
  if (head_dim < 2 || head_dim > 256 || head_dim % 2 || n_kv_heads <= 0 || n_q_heads <= 0 || n_layers <= 0 ||
      n_kv_max <= 0) {
    fprintf(stderr, "PolarQuant (HIP): init: unsupported head_dim=%d n_kv_heads=%d n_q_heads=%d n_layers=%d "
                    "n_kv_max=%d\n", head_dim, n_kv_heads, n_q_heads, n_layers, n_kv_max);
    return nullptr;
  }
  polarquant_state *st = new polarquant_state();
  memset(st, 0, sizeof(*st));
  if (n_bits != 2 && n_bits != 3 && n_bits != 4) {
    fprintf(stderr, "PolarQuant: unsupported n_bits=%d, using 4\n", n_bits);
    n_bits = 4;
  }
  st->enabled = 1;
  st->n_bits = n_bits;
  st->n_levels = 1 << n_bits;
  st->head_dim = head_dim;
  st->n_kv_heads = n_kv_heads;
  st->n_q_heads = n_q_heads;
  st->n_layers = n_layers;
  st->n_kv_max = n_kv_max;

  const float *cb = n_bits == 4 ? pqkv::kGgmlCodebook4 : n_bits == 3 ? pqkv::kGgmlCodebook3 : pqkv::kGgmlCodebook2;
  std::vector<float> R((size_t)head_dim * head_dim);
  pqkv::gram_schmidt_rotation(R.data(), head_dim, 42);
  bool ok = report(hipMalloc(&st->codebook, st->n_levels * sizeof(float)), "hipMalloc codebook") &&
            report(hipMemcpy(st->codebook, cb, st->n_levels * sizeof(float), hipMemcpyHostToDevice), "copy cb") &&
            report(hipMalloc(&st->rotation, R.size() * sizeof(float)), "hipMalloc rotation") &&
            report(hipMemcpy(st->rotation, R.data(), R.size() * sizeof(float), hipMemcpyHostToDevice), "copy R");
  st->layers = new polarquant_kv_layer[n_layers];
  memset(st->layers, 0, sizeof(polarquant_kv_layer) * n_layers);
  const size_t packed = (size_t)n_kv_heads * n_kv_max * (head_dim / 2);
  const size_t rad = (size_t)n_kv_heads * n_kv_max * sizeof(float);
  for (int l = 0; ok && l < n_layers; ++l) {
    polarquant_kv_layer &L = st->layers[l];
    ok = report(hipMalloc(&L.k_packed, packed), "hipMalloc k_packed") &&
         report(hipMalloc(&L.k_radius, rad), "hipMalloc k_radius") &&
         report(hipMalloc(&L.v_packed, packed), "hipMalloc v_packed") &&
         report(hipMalloc(&L.v_radius, rad), "hipMalloc v_radius") &&
         report(hipMemset(L.k_packed, 0, packed), "memset") && report(hipMemset(L.k_radius, 0, rad), "memset") &&
         report(hipMemset(L.v_packed, 0, packed), "memset") && report(hipMemset(L.v_radius, 0, rad), "memset");
  }
  if (!ok) {
    polarquant_free_c(st);
    return nullptr;
  }
  const double comp = (double)n_layers * 2 * n_kv_heads * n_kv_max * (head_dim / 2 + sizeof(float));
  const double orig = (double)n_layers * 2 * n_kv_heads * n_kv_max * head_dim * sizeof(float);
  fprintf(stderr, "PolarQuant-KV initialized (HIP):\n  head_dim=%d, n_kv_heads=%d, n_q_heads=%d, n_layers=%d\n"
                  "  n_bits=%d, n_levels=%d, n_kv_max=%d\n"
                  "  Compressed KV Cache: %.2f MB (original FP32: %.2f MB, ratio: %.1fx)\n",
          head_dim, n_kv_heads, n_q_heads, n_layers, st->n_bits, st->n_levels, n_kv_max, comp / (1024.0 * 1024.0),
          orig / (1024.0 * 1024.0), orig / comp);
  return st;
}

void polarquant_free_c(polarquant_state *st) {
  if (!st) return;
  if (st->codebook) (void)hipFree(st->codebook);
  if (st->rotation) (void)hipFree(st->rotation);
  if (st->layers) {
    for (int l = 0; l < st->n_layers; ++l) {
      polarquant_kv_layer &L = st->layers[l];
      if (L.k_packed) (void)hipFree(L.k_packed);
      if (L.k_radius) (void)hipFree(L.k_radius);
      if (L.v_packed) (void)hipFree(L.v_packed);
      if (L.v_radius) (void)hipFree(L.v_radius);
    }
    delete[] st->layers;
  }
  delete st;
}

void polarquant_compress_cuda_c(const float *input, const float *rotation, const float *codebook,
                                float *radius_out, uint8_t *packed_out, int N, int D, int n_levels, void *stream) {
  if (N <= 0 || D <= 0) return;
  if (D % 2 || D > 256 || n_levels < 2 || n_levels > 16) {
    fprintf(stderr, "PolarQuant (HIP): compress: unsupported D=%d n_levels=%d (even D up to 256)\n", D, n_levels);
    return;
  }
  // head dims 64 and 128: the fixed-d encoder; any other even D <= 256: the
  // generic one (same arithmetic, a 128- or 256-slot radius tree)
  if (D == 64 || D == 128)
    report(pqkv::launch_encode_soa(input, rotation, codebook, n_levels, radius_out, packed_out, N, D,
                                   (hipStream_t)stream),
           "compress launch");
  else
    report(pqkv::launch_encode_soa_generic(input, rotation, codebook, n_levels, radius_out, packed_out, N, D,
                                           (hipStream_t)stream),
           "compress launch");
}

void polarquant_rotate_query_cuda_c(const float *q_input, const float *rotation, float *q_rotated,
                                    int total_q_heads, int D, void *stream) {
  if (total_q_heads <= 0 || D <= 0) return;
  if (D > 256) {
    fprintf(stderr, "PolarQuant (HIP): rotate: unsupported D=%d (up to 256)\n", D);
    return;
  }
  if (D == 64 || D == 128)
    report(pqkv::launch_rotate(q_input, PQKV_F32, rotation, q_rotated, PQKV_F32, total_q_heads, D, 0, 1.0f,
                               (hipStream_t)stream),
           "rotate launch");
  else
    report(pqkv::launch_rotate_generic(q_input, rotation, q_rotated, total_q_heads, D, 0, (hipStream_t)stream),
           "rotate launch");
}

void polarquant_inverse_rotate_cuda_c(const float *input, const float *rotation, float *output, int total_q_heads,
                                      int D, void *stream) {
  if (total_q_heads <= 0 || D <= 0) return;
  if (D > 256) {
    fprintf(stderr, "PolarQuant (HIP): inverse rotate: unsupported D=%d (up to 256)\n", D);
    return;
  }
  if (D == 64 || D == 128)
    report(pqkv::launch_rotate(input, PQKV_F32, rotation, output, PQKV_F32, total_q_heads, D, 1, 1.0f,
                               (hipStream_t)stream),
           "inverse rotate launch");
  else
    report(pqkv::launch_rotate_generic(input, rotation, output, total_q_heads, D, 1, (hipStream_t)stream),
           "inverse rotate launch");
}

void polarquant_fused_attention_cuda_c(const float *q_rotated, const uint8_t *packed_k, const float *k_radius,
                                       const uint8_t *packed_v, const float *v_radius, const float *codebook,
                                       float *output, int total_q_heads, int total_kv_heads, int S, int D,
                                       int n_levels, float scale, void *stream) {
  if (total_q_heads <= 0 || S <= 0 || D <= 0) return;
  if (D % 8 || D > 256 || total_kv_heads <= 0 || total_q_heads % total_kv_heads || n_levels < 2 ||
      n_levels > 16) {
    fprintf(stderr, "PolarQuant (HIP): attention: unsupported Hq=%d Hkv=%d D=%d n_levels=%d (D a multiple of 8 "
                    "up to 256)\n", total_q_heads, total_kv_heads, D, n_levels);
    return;
  }
  // Stream-ordered scratch for the split partials, like the reference's
  // attention dispatcher, which allocates its temporaries per call
  // (patch:869-870); no host synchronisation.
  hipStream_t st = (hipStream_t)stream;
  if (D != 64 && D != 128) {
    // other head dims: the group kernel in its codebook mode (VALU)
    const size_t gws = pqkv_soa_attn_generic_workspace_bytes(total_q_heads, total_kv_heads, S, D);
    void *gwork = nullptr;
    if (!report(hipMallocAsync(&gwork, gws, st), "hipMallocAsync")) return;
    const int grc = pqkv_soa_attn_generic(q_rotated, packed_k, k_radius, packed_v, v_radius, codebook, n_levels,
                                          total_q_heads, total_kv_heads, S, D, scale, output, gwork, gws, stream);
    if (grc != PQKV_OK) fprintf(stderr, "PolarQuant (HIP): attention: %s\n", pqkv_last_error());
    report(hipFreeAsync(gwork, st), "hipFreeAsync");
    return;
  }
  const size_t ws = pqkv_decode_workspace_bytes(1, total_q_heads, total_kv_heads, S, D);
  void *work = nullptr;
  if (!report(hipMallocAsync(&work, ws, st), "hipMallocAsync")) return;
  const pqkv::SoaCache soa{k_radius, v_radius, n_levels};
  const int rc = pqkv::decode_attn_run(q_rotated, PQKV_F32, nullptr, packed_k, packed_v, codebook, codebook, 4, 4,
                                       nullptr, nullptr, nullptr, nullptr, 0, 1, total_q_heads, total_kv_heads, S, S,
                                       D, scale, output, PQKV_F32, work, ws, false, &soa, stream);
  if (rc != PQKV_OK) fprintf(stderr, "PolarQuant (HIP): attention: %s\n", pqkv_last_error());
  report(hipFreeAsync(work, st), "hipFreeAsync");
}

// ---- the reference's raw-pointer pybind surface (csrc/flash_turboquant.cu:180-230) ----

void turboquant_compress(int64_t input_ptr, int64_t R_ptr, int64_t cb_ptr, int64_t radius_ptr, int64_t packed_ptr,
                         int N, int D, int n_levels) {
  polarquant_compress_cuda_c((const float *)input_ptr, (const float *)R_ptr, (const float *)cb_ptr,
                             (float *)radius_ptr, (uint8_t *)packed_ptr, N, D, n_levels, nullptr);
}

void turboquant_full_attention(int64_t q_ptr, int64_t R_ptr, int64_t pk_ptr, int64_t kr_ptr, int64_t pv_ptr,
                               int64_t vr_ptr, int64_t k_cb_ptr, int64_t v_cb_ptr, int64_t out_ptr,
                               int64_t q_rot_ptr, int64_t score_ptr, int64_t attn_out_ptr, int total_heads,
                               int total_kv, int S, int D, int n_levels, float scale) {
  // As in the reference: the query is q_rot (rotated by the caller), the
  // rotated output goes to attn_out; q, R and out are not read
  // (flash_turboquant.cu:188-209). score ([total_heads][S] fp32, the
  // reference kernel's score buffer) serves as the scratch for the split
  // partials when this call's plan fits in it; otherwise a stream-ordered
  // allocation is made and released on the same stream.
  (void)q_ptr;
  (void)R_ptr;
  (void)out_ptr;
  if (total_heads <= 0 || S <= 0 || D <= 0) return;
  if (D % 8 || D > 256 || total_kv <= 0 || total_heads % total_kv || n_levels < 2 || n_levels > 16) {
    fprintf(stderr, "PolarQuant (HIP): turboquant_full_attention: unsupported heads=%d kv=%d D=%d n_levels=%d "
                    "(D a multiple of 8 up to 256)\n", total_heads, total_kv, D, n_levels);
    return;
  }
  if (D != 64 && D != 128) {
    // other head dims: the group kernel in its codebook mode; the keys and
    // values share one codebook there (k_cb), as the reference's callers pass
    void *score = (void *)score_ptr;
    const size_t need = pqkv_soa_attn_generic_workspace_bytes(total_heads, total_kv, S, D);
    const size_t have = (size_t)total_heads * S * sizeof(float);
    void *work = score;
    if (!score || (uintptr_t)score % 256 || have < need) {
      work = nullptr;
      if (!report(hipMallocAsync(&work, need, nullptr), "hipMallocAsync")) return;
    }
    const int grc = pqkv_soa_attn_generic((const float *)q_rot_ptr, (const uint8_t *)pk_ptr, (const float *)kr_ptr,
                                          (const uint8_t *)pv_ptr, (const float *)vr_ptr, (const float *)k_cb_ptr,
                                          n_levels, total_heads, total_kv, S, D, scale, (float *)attn_out_ptr, work,
                                          work == score ? have : need, nullptr);
    if (grc != PQKV_OK) fprintf(stderr, "PolarQuant (HIP): turboquant_full_attention: %s\n", pqkv_last_error());
    if (work != score) report(hipFreeAsync(work, nullptr), "hipFreeAsync");
    return;
  }
  const pqkv::SoaCache soa{(const float *)kr_ptr, (const float *)vr_ptr, n_levels};
  void *score = (void *)score_ptr;
  const size_t score_bytes = (size_t)total_heads * S * sizeof(float);
  int rc = PQKV_ERR_WORKSPACE;
  if (score && (uintptr_t)score % 16 == 0)
    rc = pqkv::decode_attn_run((const void *)q_rot_ptr, PQKV_F32, nullptr, (const uint8_t *)pk_ptr,
                               (const uint8_t *)pv_ptr, (const float *)k_cb_ptr, (const float *)v_cb_ptr, 4, 4,
                               nullptr, nullptr, nullptr, nullptr, 0, 1, total_heads, total_kv, S, S, D, scale,
                               (void *)attn_out_ptr, PQKV_F32, score, score_bytes, true, &soa, nullptr);
  if (rc == PQKV_ERR_WORKSPACE) {
    const size_t ws = pqkv_decode_workspace_bytes(1, total_heads, total_kv, S, D);
    void *work = nullptr;
    if (!report(hipMallocAsync(&work, ws, nullptr), "hipMallocAsync")) return;
    rc = pqkv::decode_attn_run((const void *)q_rot_ptr, PQKV_F32, nullptr, (const uint8_t *)pk_ptr,
                               (const uint8_t *)pv_ptr, (const float *)k_cb_ptr, (const float *)v_cb_ptr, 4, 4,
                               nullptr, nullptr, nullptr, nullptr, 0, 1, total_heads, total_kv, S, S, D, scale,
                               (void *)attn_out_ptr, PQKV_F32, work, ws, false, &soa, nullptr);
    report(hipFreeAsync(work, nullptr), "hipFreeAsync");
  }
  if (rc != PQKV_OK) fprintf(stderr, "PolarQuant (HIP): turboquant_full_attention: %s\n", pqkv_last_error());
}

}  // extern "C"
