// C ABI of libpqkv_hip.so (declared in include/pqkv.h).
//
// Every entry point validates its arguments in host code first and only then
// touches HIP, so argument errors are testable on a machine without a GPU.
#include "../../include/pqkv.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "pqkv_launch.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_status(hipError_t e, const char *what) {
  if (e == hipSuccess) return PQKV_OK;
  return fail(PQKV_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool supported_d(int d) { return d == 64 || d == 128; }

// Decode kernel choice: the matrix-core kernel serves every width pair, with
// or without QJL; PQKV_DECODE_KERNEL=valu forces the fp32 VALU kernel.
bool use_mfma() {
  const char *e = getenv("PQKV_DECODE_KERNEL");
  return !(e && strcmp(e, "valu") == 0);
}
bool supported_bits(int b) { return b == 2 || b == 4; }
bool float_dtype(int t) { return t == PQKV_F32 || t == PQKV_F16; }
size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Split-K plan: about `target` workgroups, whole 64-token tiles per wave, at
// least one tile per wave; at most 1024 splits per stream (the merge kernel's
// weight table). More target never means fewer splits, so the workspace is
// sized with the largest target any launch uses (kPlanMaxTarget).
constexpr int kPlanMaxTarget = 2048;
constexpr int kValuTarget = 512;
void decode_plan(int64_t streams, int S, int target, int *splits, int *tps) {
  if (target > kPlanMaxTarget) target = kPlanMaxTarget;
  int64_t want = (target + streams - 1) / streams;
  if (want > pqkv::kMaxSplits) want = pqkv::kMaxSplits;
  int64_t t = (S + want - 1) / want;
  if (t < 256) t = 256;
  t = (t + 63) / 64 * 64;
  *tps = (int)t;
  *splits = (int)((S + t - 1) / t);
  if (*splits < 1) *splits = 1;
}

// Compute units of the current device (cached per device; 256 if the query
// fails).
int device_cus() {
  static std::mutex mu;
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lk(mu);
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

// Workgroups resident at once for the matrix-core decode kernel: compute
// units x workgroups per CU (the kernel's launch bounds and LDS use allow
// pqkv::kMfmaBlocksPerCU), so one launch is one balanced round.
int mfma_target() { return device_cus() * pqkv::kMfmaBlocksPerCU; }

struct ProfRecord {
  std::string name;
  hipEvent_t start, stop;
  bool closed;
  int launches;   // launches between the two events (the repeat count in force)
};
std::mutex g_prof_mu;
bool g_prof_on = false;
int g_prof_repeat = 1;
std::vector<ProfRecord> g_prof;

}  // namespace

namespace pqkv {

int fail_status(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

void decode_plan_for(int64_t streams, int S, int target, int *splits, int *tps) {
  decode_plan(streams, S, target, splits, tps);
}

int device_compute_units() { return device_cus(); }

void mfma_split_plan(int64_t streams, int S, int *splits, int *tps) {
  decode_plan(streams, S > 0 ? S : 1, mfma_target(), splits, tps);
}

int prof_begin(const char *name, hipStream_t s, bool repeated) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  if (!g_prof_on) return -1;
  ProfRecord r{name, nullptr, nullptr, false, repeated ? g_prof_repeat : 1};
  if (hipEventCreate(&r.start) != hipSuccess || hipEventCreate(&r.stop) != hipSuccess) return -1;
  if (hipEventRecord(r.start, s) != hipSuccess) return -1;
  g_prof.push_back(r);
  return (int)g_prof.size() - 1;
}

int prof_repeats() {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  return g_prof_on ? g_prof_repeat : 1;
}

void prof_end(int token, hipStream_t s) {
  if (token < 0) return;
  std::lock_guard<std::mutex> lk(g_prof_mu);
  if (token < (int)g_prof.size() && hipEventRecord(g_prof[token].stop, s) == hipSuccess) g_prof[token].closed = true;
}

}  // namespace pqkv

extern "C" {

int pqkv_profile_enable(int on) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  g_prof_on = on != 0;
  return PQKV_OK;
}

int pqkv_profile_repeat(int n) {
  if (n < 1 || n > 1000) return fail(PQKV_ERR_INVALID, "profile_repeat: n=%d (1..1000)", n);
  std::lock_guard<std::mutex> lk(g_prof_mu);
  g_prof_repeat = n;
  return PQKV_OK;
}

int pqkv_profile_collect(const char *name, double *total_ms, int64_t *launches) {
  if (!name || !total_ms || !launches) return fail(PQKV_ERR_INVALID, "profile_collect: null pointer");
  std::lock_guard<std::mutex> lk(g_prof_mu);
  double tot = 0.0;
  int64_t n = 0;
  std::vector<ProfRecord> keep;
  for (auto &r : g_prof) {
    if (r.name.find(name) == std::string::npos) {
      keep.push_back(r);
      continue;
    }
    if (r.closed && hipEventSynchronize(r.stop) == hipSuccess) {
      float ms = 0.0f;
      if (hipEventElapsedTime(&ms, r.start, r.stop) == hipSuccess) {
        tot += ms;
        n += r.launches;
      }
    }
    (void)hipEventDestroy(r.start);
    (void)hipEventDestroy(r.stop);
  }
  g_prof.swap(keep);
  *total_ms = tot;
  *launches = n;
  return PQKV_OK;
}

int pqkv_profile_stream_read(const void *p, size_t bytes, uint32_t *sink, int blocks, void *stream) {
  if (!p || !sink || bytes % 16 || blocks <= 0) return fail(PQKV_ERR_INVALID, "stream_read: bad arguments");
  return hip_status(pqkv::launch_stream_read(p, bytes, sink, blocks, (hipStream_t)stream), "stream_read launch");
}

int pqkv_version(void) { return 1; }

const char *pqkv_status_string(int status) {
  switch (status) {
    case PQKV_OK: return "ok";
    case PQKV_ERR_INVALID: return "invalid argument";
    case PQKV_ERR_UNSUPPORTED: return "unsupported configuration";
    case PQKV_ERR_WORKSPACE: return "workspace too small";
    case PQKV_ERR_HIP: return "HIP error";
    default: return "unknown status";
  }
}

const char *pqkv_last_error(void) { return g_err; }

int pqkv_block_bytes(int n_bits) { return supported_bits(n_bits) ? pqkv::block_bytes(n_bits) : -1; }

int64_t pqkv_vector_bytes(int d, int n_bits) {
  if (d <= 0 || d % 32 || !supported_bits(n_bits)) return -1;
  return (int64_t)(d / 32) * pqkv::block_bytes(n_bits);
}

// ---------------------------------------------------------------------------
// Lloyd-Max codebook (host). Same iteration as lloyd_max.py:12-79; sums use
// numpy's pairwise order so the float32 results match the reference's.
// ---------------------------------------------------------------------------
static double pairwise_sum(const double *a, size_t n) {
  if (n < 8) {
    double r = 0.0;
    for (size_t i = 0; i < n; ++i) r += a[i];
    return r;
  }
  if (n <= 128) {
    double r[8];
    for (int k = 0; k < 8; ++k) r[k] = a[k];
    size_t i;
    for (i = 8; i < n - (n % 8); i += 8)
      for (int k = 0; k < 8; ++k) r[k] += a[i + k];
    double res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
    for (; i < n; ++i) res += a[i];
    return res;
  }
  size_t n2 = n / 2;
  n2 -= n2 % 8;
  return pairwise_sum(a, n2) + pairwise_sum(a + n2, n - n2);
}

int pqkv_lloyd_max_codebook(int d, int n_bits, int n_iterations, int grid_size, float *centroids,
                            float *boundaries) {
  if (d < 2 || n_bits < 1 || n_bits > 8 || n_iterations < 0 || grid_size < 2 || centroids == nullptr)
    return fail(PQKV_ERR_INVALID, "lloyd_max: bad arguments d=%d bits=%d iters=%d grid=%d", d, n_bits,
                n_iterations, grid_size);
  const int L = 1 << n_bits;
  const double alpha = (d - 1) / 2.0;
  const double sigma = 1.0 / std::sqrt((double)d);
  const double xr = 6 * sigma;
  std::vector<double> grid(grid_size), pdf(grid_size);
  const double step = (xr - (-xr)) / (double)(grid_size - 1);
  for (int i = 0; i < grid_size; ++i) grid[i] = (double)i * step + (-xr);
  grid[grid_size - 1] = xr;
  // Beta(alpha, alpha) density of t = (x + 1) / 2, times the Jacobian 1/2.
  const double lbeta = 2 * std::lgamma(alpha) - std::lgamma(2 * alpha);
  for (int i = 0; i < grid_size; ++i) {
    double t = (grid[i] + 1) / 2;
    if (t < 1e-10) t = 1e-10;
    if (t > 1 - 1e-10) t = 1 - 1e-10;
    pdf[i] = std::exp((alpha - 1) * std::log(t) + (alpha - 1) * std::log1p(-t) - lbeta) / 2;
  }
  const double norm = pairwise_sum(pdf.data(), pdf.size()) * (grid[1] - grid[0]);
  for (auto &p : pdf) p = p / norm;
  std::vector<double> c(L), bnd(L + 1, 0.0), nc(L), gw, ww;
  for (int i = 0; i < L; ++i) c[i] = L == 1 ? -xr : (double)i * ((xr - (-xr)) / (double)(L - 1)) + (-xr);
  if (L > 1) c[L - 1] = xr;
  for (int it = 0; it < n_iterations; ++it) {
    bnd[0] = -xr * 2;
    bnd[L] = xr * 2;
    for (int i = 1; i < L; ++i) bnd[i] = (c[i - 1] + c[i]) / 2;
    for (int i = 0; i < L; ++i) {
      gw.clear();
      ww.clear();
      for (int g = 0; g < grid_size; ++g)
        if (grid[g] >= bnd[i] && grid[g] < bnd[i + 1]) {
          ww.push_back(pdf[g]);
          gw.push_back(grid[g] * pdf[g]);
        }
      if (!ww.empty()) {
        const double wsum = pairwise_sum(ww.data(), ww.size());
        nc[i] = wsum > 0 ? pairwise_sum(gw.data(), gw.size()) / wsum : c[i];
      } else {
        nc[i] = c[i];
      }
    }
    c = nc;
  }
  for (int i = 0; i < L; ++i) centroids[i] = (float)c[i];
  if (boundaries)
    for (int i = 0; i <= L; ++i) boundaries[i] = (float)bnd[i];
  return PQKV_OK;
}

// ---------------------------------------------------------------------------
int pqkv_rotate(const void *x, int x_dtype, const float *R, void *y, int y_dtype, int64_t n, int d, int inverse,
                void *stream) {
  if (n < 0) return fail(PQKV_ERR_INVALID, "rotate: n=%lld < 0", (long long)n);
  if (!supported_d(d)) return fail(PQKV_ERR_UNSUPPORTED, "rotate: d=%d (supported: 64, 128)", d);
  if (!float_dtype(x_dtype) || !float_dtype(y_dtype))
    return fail(PQKV_ERR_UNSUPPORTED, "rotate: dtypes %d -> %d", x_dtype, y_dtype);
  if (n == 0) return PQKV_OK;
  if (!x || !R || !y) return fail(PQKV_ERR_INVALID, "rotate: null pointer");
  if ((uintptr_t)R % 16) return fail(PQKV_ERR_INVALID, "rotate: R must be 16-byte aligned");
  return hip_status(pqkv::launch_rotate(x, x_dtype, R, y, y_dtype, n, d, inverse ? 1 : 0, 1.0f,
                                        (hipStream_t)stream),
                    "rotate launch");
}

int pqkv_quantize_rotated(const float *x_rot, const float *codebook, int n_bits, uint8_t *blocks_out,
                          float *radius_out, int64_t n, int d, void *stream) {
  if (n < 0) return fail(PQKV_ERR_INVALID, "quantize_rotated: n < 0");
  if (!supported_d(d) || !supported_bits(n_bits))
    return fail(PQKV_ERR_UNSUPPORTED, "quantize_rotated: d=%d bits=%d", d, n_bits);
  if (n == 0) return PQKV_OK;
  if (!x_rot || !codebook || !blocks_out) return fail(PQKV_ERR_INVALID, "quantize_rotated: null pointer");
  return hip_status(pqkv::launch_quantize_rotated(x_rot, codebook, n_bits, blocks_out, radius_out, n, d,
                                                  (hipStream_t)stream),
                    "quantize_rotated launch");
}

namespace {

int encode_validate(const void *x, int x_dtype, int64_t x_outer_stride, const float *R, const float *codebook,
                    int n_bits, uint8_t *blocks, int64_t blocks_outer_stride, int64_t n_outer, int64_t n_inner, int d,
                    const float *p_rot, int m, uint8_t *qjl, int64_t qjl_outer_stride) {
  if (n_outer < 0 || n_inner < 0) return fail(PQKV_ERR_INVALID, "encode: negative count");
  if (!supported_d(d) || !supported_bits(n_bits))
    return fail(PQKV_ERR_UNSUPPORTED, "encode: d=%d bits=%d", d, n_bits);
  if (!float_dtype(x_dtype) && x_dtype != PQKV_BF16) return fail(PQKV_ERR_UNSUPPORTED, "encode: x dtype %d", x_dtype);
  if ((qjl == nullptr) != (p_rot == nullptr)) return fail(PQKV_ERR_INVALID, "encode: qjl and p_rot go together");
  if (qjl && m != d) return fail(PQKV_ERR_UNSUPPORTED, "encode: QJL needs m == d (m=%d, d=%d)", m, d);
  if (n_outer * n_inner == 0) return PQKV_OK;
  if (!x || !R || !codebook || !blocks) return fail(PQKV_ERR_INVALID, "encode: null pointer");
  const int64_t vb = pqkv_vector_bytes(d, n_bits);
  if (n_outer > 1 && (x_outer_stride < n_inner * d || blocks_outer_stride < n_inner * vb))
    return fail(PQKV_ERR_INVALID, "encode: outer strides overlap rows");
  if (qjl && n_outer > 1 && qjl_outer_stride < n_inner * (m / 8))
    return fail(PQKV_ERR_INVALID, "encode: qjl outer stride overlaps rows");
  return 1;  // valid, work to do
}

// The matrix-core encoder takes fp16 input whose rows and R (and P_rot) allow
// 16-byte loads, and blocks (and signs) that allow dword stores.
bool fast_encode_ok(const void *x, int x_dtype, int64_t x_outer_stride, int64_t n_outer, int64_t n_inner,
                    const float *R, const float *p_rot, const uint8_t *qjl, int64_t qjl_outer_stride,
                    const uint8_t *blocks, int64_t blocks_outer_stride) {
  if (x_dtype != PQKV_F16) return false;
  if ((uintptr_t)x % 16 || (uintptr_t)R % 16 || (uintptr_t)blocks % 4) return false;
  if (qjl != nullptr && ((uintptr_t)p_rot % 16 || (uintptr_t)qjl % 4)) return false;
  if (n_outer * n_inner > ((int64_t)1 << 32) - 64) return false;  // 32-bit vector indices
  return n_outer <= 1 || (x_outer_stride % 8 == 0 && blocks_outer_stride % 4 == 0 &&
                          (qjl == nullptr || qjl_outer_stride % 4 == 0));
}

// Rows that follow each other with no gap in x, the blocks and the signs are
// one run of vectors: a single row lets the kernels skip the row split.
pqkv::EncodeArgs encode_args(const void *x, int64_t x_outer_stride, const float *R, const float *codebook,
                             int n_bits, uint8_t *blocks, int64_t blocks_outer_stride, int64_t n_outer,
                             int64_t n_inner, int d, const float *p_rot, int m, uint8_t *qjl,
                             int64_t qjl_outer_stride) {
  const int64_t vb = pqkv_vector_bytes(d, n_bits);
  if (n_outer > 1 && x_outer_stride == n_inner * d && blocks_outer_stride == n_inner * vb &&
      (qjl == nullptr || qjl_outer_stride == n_inner * (m / 8))) {
    n_inner *= n_outer;
    n_outer = 1;
  }
  return pqkv::EncodeArgs{x, x_outer_stride, R, codebook, n_bits, blocks, blocks_outer_stride, n_outer, n_inner,
                          d, p_rot, m, qjl, qjl_outer_stride};
}

}  // namespace

// Encoder choice: the matrix-core encoder wherever fast_encode_ok holds;
// PQKV_ENCODE_KERNEL=exact forces the FMA-chain encoder (the reference
// kernel's rotation rounding) everywhere.
int pqkv_encode(const void *x, int x_dtype, int64_t x_outer_stride, const float *R, const float *codebook,
                int n_bits, uint8_t *blocks, int64_t blocks_outer_stride, int64_t n_outer, int64_t n_inner, int d,
                const float *p_rot, int m, uint8_t *qjl, int64_t qjl_outer_stride, void *stream) {
  const int v = encode_validate(x, x_dtype, x_outer_stride, R, codebook, n_bits, blocks, blocks_outer_stride, n_outer,
                                n_inner, d, p_rot, m, qjl, qjl_outer_stride);
  if (v <= 0) return v;
  const pqkv::EncodeArgs a = encode_args(x, x_outer_stride, R, codebook, n_bits, blocks, blocks_outer_stride,
                                         n_outer, n_inner, d, p_rot, m, qjl, qjl_outer_stride);
  const char *env = getenv("PQKV_ENCODE_KERNEL");
  const bool exact = env && strcmp(env, "exact") == 0;
  hipError_t e;
  if (!exact && fast_encode_ok(x, x_dtype, x_outer_stride, n_outer, n_inner, R, p_rot, qjl, qjl_outer_stride, blocks,
                                 blocks_outer_stride)) {
    const int tok = pqkv::prof_begin("encode_mfma", (hipStream_t)stream, true);
    e = hipSuccess;
    for (int rep = 0, nrep = pqkv::prof_repeats(); rep < nrep && e == hipSuccess; ++rep)
      e = pqkv::launch_encode_mfma(a, nullptr, nullptr, device_cus(), (hipStream_t)stream);
    pqkv::prof_end(tok, (hipStream_t)stream);
  } else {
    const int tok = pqkv::prof_begin("encode_exact", (hipStream_t)stream, true);
    e = hipSuccess;
    for (int rep = 0, nrep = pqkv::prof_repeats(); rep < nrep && e == hipSuccess; ++rep)
      e = pqkv::launch_encode_exact(a, x_dtype, (hipStream_t)stream);
    pqkv::prof_end(tok, (hipStream_t)stream);
  }
  return hip_status(e, "encode launch");
}

int pqkv_encode_mfma(const void *x, int x_dtype, int64_t x_outer_stride, const float *R, const float *codebook,
                     int n_bits, uint8_t *blocks, int64_t blocks_outer_stride, int64_t n_outer, int64_t n_inner,
                     int d, float *rot_out, float *radius_out, void *stream) {
  const int v = encode_validate(x, x_dtype, x_outer_stride, R, codebook, n_bits, blocks, blocks_outer_stride, n_outer,
                                n_inner, d, nullptr, 0, nullptr, 0);
  if (v <= 0) return v;
  if (!fast_encode_ok(x, x_dtype, x_outer_stride, n_outer, n_inner, R, nullptr, nullptr, 0, blocks,
                      blocks_outer_stride))
    return fail(PQKV_ERR_UNSUPPORTED,
                "encode_mfma: needs fp16 x, 16-byte aligned x rows and R, 4-byte aligned blocks, < 2^32 vectors");
  const pqkv::EncodeArgs a = encode_args(x, x_outer_stride, R, codebook, n_bits, blocks, blocks_outer_stride,
                                         n_outer, n_inner, d, nullptr, 0, nullptr, 0);
  const int tok = pqkv::prof_begin("encode_mfma", (hipStream_t)stream);
  const hipError_t e = pqkv::launch_encode_mfma(a, rot_out, radius_out, device_cus(), (hipStream_t)stream);
  pqkv::prof_end(tok, (hipStream_t)stream);
  return hip_status(e, "encode_mfma launch");
}

size_t pqkv_decode_workspace_bytes(int B, int Hq, int Hkv, int S, int d) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || S < 0 || d <= 0) return 0;
  int splits = 1, tps = 0;
  // bound over every plan a call can make: fewest streams per launch (B),
  // largest target
  decode_plan(B, S > 0 ? S : 1, kPlanMaxTarget, &splits, &tps);
  return pqkv::decode_workspace_layout(B, Hq, splits, d, nullptr, nullptr, nullptr);
}

int pqkv_decode_attn(const void *q, int q_dtype, const float *R, const uint8_t *k_cache, const uint8_t *v_cache,
                     const float *k_codebooks, const float *v_codebooks, int k_bits, int v_bits,
                     const int *k_head_bits, const int *v_head_bits, const uint8_t *qjl_signs, const float *p_rot,
                     int m, int B, int Hq, int Hkv, int S, int S_max, int d, float scale, void *out, int out_dtype,
                     void *workspace, size_t workspace_bytes, void *stream) {
  return pqkv::decode_attn_run(q, q_dtype, R, k_cache, v_cache, k_codebooks, v_codebooks, k_bits, v_bits,
                               k_head_bits, v_head_bits, qjl_signs, p_rot, m, B, Hq, Hkv, S, S_max, d, scale, out,
                               out_dtype, workspace, workspace_bytes, false, nullptr, stream);
}


int pqkv_group_compress(const void *x, int x_dtype, const double *R, int64_t n, int d, int n_bits, int group_size,
                        float *radius, uint8_t *codes, float *mins, float *scales, void *stream) {
  if (n < 0) return fail(PQKV_ERR_INVALID, "group_compress: n < 0");
  if (d < 1 || d > 256) return fail(PQKV_ERR_UNSUPPORTED, "group_compress: d=%d (1..256)", d);
  if (n_bits < 2 || n_bits > 8) return fail(PQKV_ERR_INVALID, "group_compress: n_bits=%d (2..8)", n_bits);
  if (group_size < 1 || group_size > d)
    return fail(PQKV_ERR_INVALID, "group_compress: group_size=%d (1..d=%d)", group_size, d);
  if (x_dtype != PQKV_F32 && x_dtype != PQKV_F16) return fail(PQKV_ERR_UNSUPPORTED, "group_compress: x dtype");
  if (n == 0) return PQKV_OK;
  if (!x || !R || !radius || !codes || !mins || !scales) return fail(PQKV_ERR_INVALID, "group_compress: null pointer");
  return hip_status(pqkv::launch_group_compress(x, x_dtype, R, n, d, n_bits, group_size, radius, codes, mins, scales,
                                                (hipStream_t)stream),
                    "group_compress launch");
}

int pqkv_group_decompress(const float *radius, const uint8_t *codes, const float *mins, const float *scales,
                          const double *R, int64_t n, int d, int group_size, float *out, void *stream) {
  if (n < 0) return fail(PQKV_ERR_INVALID, "group_decompress: n < 0");
  if (d < 1 || d > 256) return fail(PQKV_ERR_UNSUPPORTED, "group_decompress: d=%d (1..256)", d);
  if (group_size < 1 || group_size > d)
    return fail(PQKV_ERR_INVALID, "group_decompress: group_size=%d (1..d=%d)", group_size, d);
  if (n == 0) return PQKV_OK;
  if (!radius || !codes || !mins || !scales || !R || !out)
    return fail(PQKV_ERR_INVALID, "group_decompress: null pointer");
  return hip_status(pqkv::launch_group_decompress(radius, codes, mins, scales, R, n, d, group_size, out,
                                                  (hipStream_t)stream),
                    "group_decompress launch");
}

size_t pqkv_decode_segments_workspace_bytes(int B, int Hq, int Hkv, int n_seg, const int *S, int d) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || d <= 0 || n_seg < 1 || n_seg > PQKV_MAX_SEGMENTS || !S) return 0;
  for (int i = 0; i < n_seg; ++i)
    if (S[i] < 0) return 0;
  int splits[PQKV_MAX_SEGMENTS], tps[PQKV_MAX_SEGMENTS];
  // bound over the plans a call can make (largest target)
  const int total = pqkv::segment_plans(B, Hkv, n_seg, S, kPlanMaxTarget, splits, tps);
  return pqkv::decode_workspace_layout(B, Hq, total > 0 ? total : 1, d, nullptr, nullptr, nullptr);
}

int pqkv_decode_attn_segments(const void *q, int q_dtype, const float *R, int n_seg, const uint8_t *const *k_caches,
                              const uint8_t *const *v_caches, const float *const *k_codebooks,
                              const float *const *v_codebooks, const int *k_bits, const int *v_bits, const int *S,
                              const int *S_max, int B, int Hq, int Hkv, int d, float scale, void *out, int out_dtype,
                              void *workspace, size_t workspace_bytes, void *stream) {
  return pqkv::decode_segments_run(q, q_dtype, R, n_seg, k_caches, v_caches, k_codebooks, v_codebooks, k_bits, v_bits,
                                   S, S_max, B, Hq, Hkv, d, scale, out, out_dtype, workspace, workspace_bytes, stream);
}
}  // extern "C"

namespace pqkv {

int report_hip_error(hipError_t e, const char *what) { return hip_status(e, what); }

// Workspace of one decode call with `splits` partitions per stream: rotated
// queries, split partials, and the QJL projections P_rot q_rot / m, each
// 256-byte aligned. Returns the total; the nullable pointers receive the
// offsets.
size_t decode_workspace_layout(int B, int Hq, int splits, int d, size_t *q_off, size_t *part_off, size_t *pq_off) {
  const size_t q = align256((size_t)B * Hq * d * 4);
  const size_t part = align256((size_t)B * Hq * splits * (d + 2) * 4);
  if (q_off) *q_off = 0;
  if (part_off) *part_off = q;
  if (pq_off) *pq_off = q + part;
  return q + part + align256((size_t)B * Hq * d * 4);
}

// One decode call. With plan_sized the workspace need is this call's own
// split plan (the allocation-free entry point, whose scratch has a fixed
// size); otherwise it is the pqkv_decode_workspace_bytes bound the header
// promises. No allocation of any kind happens here: per-head tables live in
// fixed arrays (mixed widths are limited to PQKV_MAX_HEADS kv heads).
int decode_attn_run(const void *q, int q_dtype, const float *R, const uint8_t *k_cache, const uint8_t *v_cache,
                    const float *k_codebooks, const float *v_codebooks, int k_bits, int v_bits,
                    const int *k_head_bits, const int *v_head_bits, const uint8_t *qjl_signs, const float *p_rot,
                    int m, int B, int Hq, int Hkv, int S, int S_max, int d, float scale, void *out, int out_dtype,
                    void *workspace, size_t workspace_bytes, bool plan_sized, const SoaCache *soa,
                    void *stream, const PagedCache *pg) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || S < 0 || S_max < S)
    return fail(PQKV_ERR_INVALID, "decode: B=%d Hq=%d Hkv=%d S=%d S_max=%d", B, Hq, Hkv, S, S_max);
  if (Hq % Hkv) return fail(PQKV_ERR_INVALID, "decode: Hq=%d not a multiple of Hkv=%d", Hq, Hkv);
  if (!supported_d(d)) return fail(PQKV_ERR_UNSUPPORTED, "decode: d=%d", d);
  if (!float_dtype(q_dtype) || !float_dtype(out_dtype)) return fail(PQKV_ERR_UNSUPPORTED, "decode: dtype");
  const bool mixed = k_head_bits != nullptr || v_head_bits != nullptr;
  if (mixed && Hkv > kMaxListHeads)
    return fail(PQKV_ERR_UNSUPPORTED, "decode: mixed widths support at most %d kv heads", kMaxListHeads);
  if (!supported_bits(k_bits) && !k_head_bits) return fail(PQKV_ERR_UNSUPPORTED, "decode: k_bits=%d", k_bits);
  if (!supported_bits(v_bits) && !v_head_bits) return fail(PQKV_ERR_UNSUPPORTED, "decode: v_bits=%d", v_bits);
  int kb[kMaxListHeads], vb[kMaxListHeads];
  if (mixed)
    for (int h = 0; h < Hkv; ++h) {
      kb[h] = k_head_bits ? k_head_bits[h] : k_bits;
      vb[h] = v_head_bits ? v_head_bits[h] : v_bits;
      if (!supported_bits(kb[h]) || !supported_bits(vb[h]))
        return fail(PQKV_ERR_UNSUPPORTED, "decode: head %d widths k=%d v=%d", h, kb[h], vb[h]);
    }
  // QJL signs: an array, or (paged) sign pages
  const bool has_qjl = qjl_signs != nullptr || (pg && pg->s_pages != nullptr);
  if (has_qjl != (p_rot != nullptr)) return fail(PQKV_ERR_INVALID, "decode: qjl and p_rot go together");
  if (has_qjl && m != d) return fail(PQKV_ERR_UNSUPPORTED, "decode: QJL needs m == d");
  if (!(scale > 0.0f) || !std::isfinite(scale)) return fail(PQKV_ERR_INVALID, "decode: scale must be > 0");
  if (pg && (mixed || soa || k_bits != v_bits))
    return fail(PQKV_ERR_UNSUPPORTED, "decode: paged caches take uniform widths with k_bits == v_bits");
  if (!q || (!R && !soa) || !out) return fail(PQKV_ERR_INVALID, "decode: null pointer");
  if ((uintptr_t)R % 16) return fail(PQKV_ERR_INVALID, "decode: R must be 16-byte aligned");
  if (soa && (mixed || k_bits != 4 || v_bits != 4 || qjl_signs || soa->levels < 1 || soa->levels > 16 ||
              (S > 0 && (!soa->k_rad || !soa->v_rad))))
    return fail(PQKV_ERR_UNSUPPORTED, "decode: the SoA layout takes 4-bit codes and no QJL signs");
  if ((uintptr_t)p_rot % 16) return fail(PQKV_ERR_INVALID, "decode: p_rot must be 16-byte aligned");
  if (S > 0 && (pg ? (!pg->k_pages || !pg->v_pages) : (!k_cache || !v_cache)))
    return fail(PQKV_ERR_INVALID, "decode: null cache");
  if (S > 0 && (!k_codebooks || !v_codebooks)) return fail(PQKV_ERR_INVALID, "decode: null codebook");

  // One split plan serves every launch (they share the partials layout); it
  // is sized for the largest launch: all kv heads, or with mixed widths the
  // largest group of heads sharing (k bits, v bits). Heads that are all 4/4
  // (one shared codebook) or 2/2 run as one launch.
  // (the paged and SoA modes exist only in the matrix-core kernel)
  const bool mfma = use_mfma() || soa != nullptr || pg != nullptr;
  int group = Hkv;
  bool pair = false;
  if (mixed) {
    int count[2][2] = {{0, 0}, {0, 0}};
    for (int h = 0; h < Hkv; ++h) ++count[kb[h] == 4][vb[h] == 4];
    pair = mfma && count[1][1] > 0 && count[0][0] > 0 && count[1][0] == 0 && count[0][1] == 0 &&
           k_codebooks == v_codebooks;
    if (!pair) group = std::max(std::max(count[0][0], count[0][1]), std::max(count[1][0], count[1][1]));
  }
  int splits = 1, tps = 0;
  decode_plan((int64_t)B * group, S > 0 ? S : 1, mfma ? mfma_target() : kValuTarget, &splits, &tps);
  size_t q_off, part_off, pq_off;
  const size_t plan_need = decode_workspace_layout(B, Hq, splits, d, &q_off, &part_off, &pq_off);
  if (S > 0) {
    const size_t need = plan_sized ? plan_need : pqkv_decode_workspace_bytes(B, Hq, Hkv, S, d);
    if (plan_sized && (!workspace || workspace_bytes < need))
      return fail(PQKV_ERR_WORKSPACE,
                  "decode: this call's split plan needs %zu bytes of scratch, more than the %zu available "
                  "(pqkv_decode_attn takes a caller workspace of any size)", need, workspace_bytes);
    if (!workspace || workspace_bytes < need)
      return fail(PQKV_ERR_WORKSPACE, "decode: workspace %zu < %zu bytes", workspace_bytes, need);
  }
  hipStream_t st = (hipStream_t)stream;
  if (S == 0) {
    const size_t ob = (size_t)B * Hq * d * (out_dtype == PQKV_F32 ? 4 : 2);
    return hip_status(launch_fill_zero(out, ob, st), "decode zero fill");
  }
  float *q32 = (float *)((char *)workspace + q_off);
  float *part = (float *)((char *)workspace + part_off);
  float *pq32 = (float *)((char *)workspace + pq_off);
  const float kLog2e = 1.4426950408889634f;
  int tok = prof_begin("decode_rotate", st, true);
  hipError_t e = hipSuccess;
  for (int rep = 0, nrep = prof_repeats(); rep < nrep && e == hipSuccess; ++rep)
    // QJL: the projections P_rot q_rot / m (m == d) come from the same launch
    e = has_qjl ? launch_rotate2(q, q_dtype, R, p_rot, q32, pq32, (int64_t)B * Hq, d, scale * kLog2e,
                                 1.0f / (float)m, st)
                  : launch_rotate(q, q_dtype, R, q32, PQKV_F32, (int64_t)B * Hq, d, 0, scale * kLog2e, st);
  prof_end(tok, st);
  if (e != hipSuccess) return hip_status(e, "decode query rotation");

  DecodeArgs a;
  memset(&a, 0, sizeof(a));
  a.q = q32;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.k_cb = k_codebooks;
  a.v_cb = v_codebooks;
  a.cb_head_stride = mixed ? 16 : 0;
  a.cb_levels = soa ? soa->levels : 16;
  a.k_rad = soa ? soa->k_rad : nullptr;
  a.v_rad = soa ? soa->v_rad : nullptr;
  a.qjl = qjl_signs;
  a.p_rot = p_rot;
  a.pq = has_qjl ? pq32 : nullptr;
  a.part = part;
  if (pg) {
    a.k_pages = pg->k_pages;
    a.v_pages = pg->v_pages;
    a.s_pages = pg->s_pages;
    a.page_shift = pg->page_shift;
    a.max_pages = pg->max_pages;
  }
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.gq = Hq / Hkv;
  a.S = S;
  a.S_max = S_max;
  a.d = d;
  a.splits = splits;
  a.tokens_per_split = tps;
  a.split_base = 0;
  a.split_stride = splits;

  // Query heads of a kv head in launches of at most kMaxGroup (the matrix
  // tile holds 8 heads): the group is cut into equal parts where it divides,
  // the first ones one head larger otherwise.
  const int n_sub = (a.gq + kMaxGroup - 1) / kMaxGroup;
  auto for_each_subgroup = [&](auto &&launch) -> hipError_t {
    int off = 0;
    for (int i = 0; i < n_sub; ++i) {
      const int g = a.gq / n_sub + (i < a.gq % n_sub ? 1 : 0);
      hipError_t r = launch(off, g);
      if (r != hipSuccess) return r;
      off += g;
    }
    return hipSuccess;
  };

  if (!mixed) {
    const int64_t kvb = soa ? d / 2 : pqkv_vector_bytes(d, k_bits), vvb = soa ? d / 2 : pqkv_vector_bytes(d, v_bits);
    a.k_head_stride = (int64_t)S_max * kvb;
    a.v_head_stride = (int64_t)S_max * vvb;
    a.k_batch_stride = a.k_head_stride * Hkv;
    a.v_batch_stride = a.v_head_stride * Hkv;
    a.n_heads = Hkv;
    a.listed = 0;
    e = for_each_subgroup([&](int off, int g) {
      a.q_off = off;
      a.g = g;
      const int t = prof_begin("decode_split", st, true);
      hipError_t r = hipSuccess;
      for (int rep = 0, nrep = prof_repeats(); rep < nrep && r == hipSuccess; ++rep)
        r = pg     ? launch_decode_mfma_paged(a, k_bits, st)
            : soa  ? launch_decode_mfma_soa(a, st)
            : mfma ? launch_decode_mfma(a, k_bits, v_bits, st)
                   : launch_decode_split(a, k_bits, v_bits, st);
      prof_end(t, st);
      return r;
    });
    if (e != hipSuccess) return hip_status(e, "decode split launch");
  } else {
    // Per-(b, h) runs of S_max vectors of the head's own width, (b, h) order.
    int64_t koff[kMaxListHeads + 1], voff[kMaxListHeads + 1];
    koff[0] = voff[0] = 0;
    for (int h = 0; h < Hkv; ++h) {
      koff[h + 1] = koff[h] + (int64_t)S_max * pqkv_vector_bytes(d, kb[h]);
      voff[h + 1] = voff[h] + (int64_t)S_max * pqkv_vector_bytes(d, vb[h]);
    }
    a.k_batch_stride = koff[Hkv];
    a.v_batch_stride = voff[Hkv];
    a.listed = 1;
    if (pair) {
      DecodeArgs a2 = a;
      int n4 = 0, n2 = 0;
      for (int h = 0; h < Hkv; ++h) {
        DecodeArgs &gr = kb[h] == 4 ? a : a2;
        int &n = kb[h] == 4 ? n4 : n2;
        gr.heads[n] = (int16_t)h;
        gr.k_head_off[n] = koff[h];
        gr.v_head_off[n] = voff[h];
        ++n;
      }
      a.n_heads = n4;
      a2.n_heads = n2;
      e = for_each_subgroup([&](int off, int g) {
        a.q_off = a2.q_off = off;
        a.g = a2.g = g;
        const int t = prof_begin("decode_split", st, true);
        hipError_t r = hipSuccess;
        for (int rep = 0, nrep = prof_repeats(); rep < nrep && r == hipSuccess; ++rep)
          r = launch_decode_mfma_pair(a, a2, st);
        prof_end(t, st);
        return r;
      });
      if (e != hipSuccess) return hip_status(e, "decode split launch");
    } else {
      for (int kbits : {4, 2})
        for (int vbits : {4, 2}) {
          int n = 0;
          for (int h = 0; h < Hkv; ++h)
            if (kb[h] == kbits && vb[h] == vbits) {
              a.heads[n] = (int16_t)h;
              a.k_head_off[n] = koff[h];
              a.v_head_off[n] = voff[h];
              ++n;
            }
          if (n == 0) continue;
          a.n_heads = n;
          e = for_each_subgroup([&](int off, int g) {
            a.q_off = off;
            a.g = g;
            const int t = prof_begin("decode_split", st, true);
            hipError_t r = hipSuccess;
            for (int rep = 0, nrep = prof_repeats(); rep < nrep && r == hipSuccess; ++rep)
              r = mfma ? launch_decode_mfma(a, kbits, vbits, st) : launch_decode_split(a, kbits, vbits, st);
            prof_end(t, st);
            return r;
          });
          if (e != hipSuccess) return hip_status(e, "decode split launch");
        }
    }
  }
  tok = prof_begin("decode_merge", st, true);
  for (int rep = 0, nrep = prof_repeats(); rep < nrep && e == hipSuccess; ++rep)
    e = launch_decode_merge(part, R, out, out_dtype, B * Hq, splits, d, st);
  prof_end(tok, st);
  return hip_status(e, "decode merge launch");
}

// Split plans of the segments of a segmented decode call (B * Hkv streams
// of S[i] tokens each); returns the total, the partials per query head that
// the plans share.
int segment_plans(int B, int Hkv, int n_seg, const int *S, int target, int *splits, int *tps) {
  int total = 0;
  for (int i = 0; i < n_seg; ++i) {
    splits[i] = 0;
    tps[i] = 0;
    if (S[i] > 0) {
      decode_plan((int64_t)B * Hkv, S[i], target, &splits[i], &tps[i]);
      total += splits[i];
    }
  }
  return total;
}

// Decode attention over segments of one logical cache: one query rotation,
// each segment's split launches writing partials split_base .. of one
// layout, one merge over all of them.
int decode_segments_run(const void *q, int q_dtype, const float *R, int n_seg, const uint8_t *const *k_caches,
                        const uint8_t *const *v_caches, const float *const *k_codebooks,
                        const float *const *v_codebooks, const int *k_bits, const int *v_bits, const int *S,
                        const int *S_max, int B, int Hq, int Hkv, int d, float scale, void *out, int out_dtype,
                        void *workspace, size_t workspace_bytes, void *stream) {
  if (n_seg < 1 || n_seg > PQKV_MAX_SEGMENTS)
    return fail(PQKV_ERR_UNSUPPORTED, "decode segments: %d segments (1..%d)", n_seg, PQKV_MAX_SEGMENTS);
  if (!k_caches || !v_caches || !k_codebooks || !v_codebooks || !k_bits || !v_bits || !S || !S_max)
    return fail(PQKV_ERR_INVALID, "decode segments: null segment array");
  if (B <= 0 || Hq <= 0 || Hkv <= 0) return fail(PQKV_ERR_INVALID, "decode segments: B=%d Hq=%d Hkv=%d", B, Hq, Hkv);
  if (Hq % Hkv) return fail(PQKV_ERR_INVALID, "decode segments: Hq=%d not a multiple of Hkv=%d", Hq, Hkv);
  if (!supported_d(d)) return fail(PQKV_ERR_UNSUPPORTED, "decode segments: d=%d", d);
  if (!float_dtype(q_dtype) || !float_dtype(out_dtype)) return fail(PQKV_ERR_UNSUPPORTED, "decode segments: dtype");
  if (!(scale > 0.0f) || !std::isfinite(scale)) return fail(PQKV_ERR_INVALID, "decode segments: scale must be > 0");
  if (!q || !R || !out) return fail(PQKV_ERR_INVALID, "decode segments: null pointer");
  if ((uintptr_t)R % 16) return fail(PQKV_ERR_INVALID, "decode segments: R must be 16-byte aligned");
  for (int i = 0; i < n_seg; ++i) {
    if (S[i] < 0 || S_max[i] < S[i])
      return fail(PQKV_ERR_INVALID, "decode segments: segment %d S=%d S_max=%d", i, S[i], S_max[i]);
    if (!supported_bits(k_bits[i]) || !supported_bits(v_bits[i]))
      return fail(PQKV_ERR_UNSUPPORTED, "decode segments: segment %d widths k=%d v=%d", i, k_bits[i], v_bits[i]);
    if (S[i] > 0 && (!k_caches[i] || !v_caches[i] || !k_codebooks[i] || !v_codebooks[i]))
      return fail(PQKV_ERR_INVALID, "decode segments: segment %d null cache or codebook", i);
  }
  const bool mfma = use_mfma();
  int splits[PQKV_MAX_SEGMENTS], tps[PQKV_MAX_SEGMENTS];
  const int total = segment_plans(B, Hkv, n_seg, S, mfma ? mfma_target() : kValuTarget, splits, tps);
  hipStream_t st = (hipStream_t)stream;
  if (total == 0) {
    const size_t ob = (size_t)B * Hq * d * (out_dtype == PQKV_F32 ? 4 : 2);
    return hip_status(launch_fill_zero(out, ob, st), "decode segments zero fill");
  }
  if (total > kMaxSplits)
    return fail(PQKV_ERR_UNSUPPORTED, "decode segments: %d split partials per query head (at most %d)", total,
                kMaxSplits);
  size_t q_off, part_off;
  decode_workspace_layout(B, Hq, total, d, &q_off, &part_off, nullptr);
  const size_t need = pqkv_decode_segments_workspace_bytes(B, Hq, Hkv, n_seg, S, d);
  if (!workspace || workspace_bytes < need)
    return fail(PQKV_ERR_WORKSPACE, "decode segments: workspace %zu < %zu bytes", workspace_bytes, need);
  float *q32 = (float *)((char *)workspace + q_off);
  float *part = (float *)((char *)workspace + part_off);
  const float kLog2e = 1.4426950408889634f;
  int tok = prof_begin("decode_rotate", st);
  hipError_t e = launch_rotate(q, q_dtype, R, q32, PQKV_F32, (int64_t)B * Hq, d, 0, scale * kLog2e, st);
  prof_end(tok, st);
  if (e != hipSuccess) return hip_status(e, "decode segments query rotation");
  int base = 0;
  for (int i = 0; i < n_seg; ++i) {
    if (S[i] == 0) continue;
    DecodeArgs a;
    memset(&a, 0, sizeof(a));
    a.q = q32;
    a.k_cache = k_caches[i];
    a.v_cache = v_caches[i];
    a.k_cb = k_codebooks[i];
    a.v_cb = v_codebooks[i];
    a.cb_levels = 16;
    a.part = part;
    a.B = B;
    a.Hq = Hq;
    a.Hkv = Hkv;
    a.gq = Hq / Hkv;
    a.S = S[i];
    a.S_max = S_max[i];
    a.d = d;
    a.splits = splits[i];
    a.tokens_per_split = tps[i];
    a.split_base = base;
    a.split_stride = total;
    a.k_head_stride = (int64_t)S_max[i] * pqkv_vector_bytes(d, k_bits[i]);
    a.v_head_stride = (int64_t)S_max[i] * pqkv_vector_bytes(d, v_bits[i]);
    a.k_batch_stride = a.k_head_stride * Hkv;
    a.v_batch_stride = a.v_head_stride * Hkv;
    a.n_heads = Hkv;
    // query heads of a kv head in launches of at most kMaxGroup, as in
    // decode_attn_run
    const int n_sub = (a.gq + kMaxGroup - 1) / kMaxGroup;
    int off = 0;
    for (int j = 0; j < n_sub; ++j) {
      a.q_off = off;
      a.g = a.gq / n_sub + (j < a.gq % n_sub ? 1 : 0);
      const int t = prof_begin("decode_split", st);
      e = mfma ? launch_decode_mfma(a, k_bits[i], v_bits[i], st) : launch_decode_split(a, k_bits[i], v_bits[i], st);
      prof_end(t, st);
      if (e != hipSuccess) return hip_status(e, "decode segments split launch");
      off += a.g;
    }
    base += splits[i];
  }
  tok = prof_begin("decode_merge", st);
  e = launch_decode_merge(part, R, out, out_dtype, B * Hq, total, d, st);
  prof_end(tok, st);
  return hip_status(e, "decode segments merge launch");
}

}  // namespace pqkv

extern "C" {

size_t pqkv_prefill_workspace_bytes(int B, int Hq, int Hkv, int Sq, int S, int d) {
  (void)Hkv;
  (void)S;
  if (B <= 0 || Hq <= 0 || Sq <= 0 || d <= 0) return 0;
  // rotated queries, rotated outputs and (QJL) the projections P_rot q_rot / m,
  // fp32 [B][Hq][Sq][d] each
  return 3 * align256((size_t)B * Hq * Sq * d * 4);
}

int pqkv_prefill_attn(const void *q, int q_dtype, const float *R, const uint8_t *k_cache, const uint8_t *v_cache,
                      const float *k_codebooks, const float *v_codebooks, int k_bits, int v_bits,
                      const int *k_head_bits, const int *v_head_bits, const uint8_t *qjl_signs, const float *p_rot,
                      int m, int B, int Hq, int Hkv, int Sq, int q_start, int S, int S_max, int d, float scale,
                      int causal, void *out, int out_dtype, void *workspace, size_t workspace_bytes, void *stream) {
  return pqkv::prefill_attn_run(q, q_dtype, R, k_cache, v_cache, k_codebooks, v_codebooks, k_bits, v_bits,
                                k_head_bits, v_head_bits, qjl_signs, p_rot, m, B, Hq, Hkv, Sq, q_start, S, S_max, d,
                                scale, causal, out, out_dtype, workspace, workspace_bytes, stream, nullptr);
}

}  // extern "C"

namespace pqkv {

int prefill_attn_run(const void *q, int q_dtype, const float *R, const uint8_t *k_cache, const uint8_t *v_cache,
                     const float *k_codebooks, const float *v_codebooks, int k_bits, int v_bits,
                     const int *k_head_bits, const int *v_head_bits, const uint8_t *qjl_signs, const float *p_rot,
                     int m, int B, int Hq, int Hkv, int Sq, int q_start, int S, int S_max, int d, float scale,
                     int causal, void *out, int out_dtype, void *workspace, size_t workspace_bytes, void *stream,
                     const PagedCache *pg) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || Sq < 0 || S < 0 || S_max < S || q_start < 0)
    return fail(PQKV_ERR_INVALID, "prefill: B=%d Hq=%d Hkv=%d Sq=%d S=%d S_max=%d q_start=%d", B, Hq, Hkv, Sq, S,
                S_max, q_start);
  if (Hq % Hkv) return fail(PQKV_ERR_INVALID, "prefill: Hq=%d not a multiple of Hkv=%d", Hq, Hkv);
  const bool qjl = qjl_signs != nullptr || (pg && pg->s_pages != nullptr);
  if (Hq / Hkv > pqkv::prefill_rows_per_block(qjl))
    return fail(PQKV_ERR_UNSUPPORTED, "prefill: group size %d", Hq / Hkv);
  if (causal && (int64_t)q_start + Sq > S)
    return fail(PQKV_ERR_INVALID, "prefill: causal queries at %d..%d are not all in the cache (S=%d)", q_start,
                q_start + Sq - 1, S);
  if (!supported_d(d)) return fail(PQKV_ERR_UNSUPPORTED, "prefill: d=%d", d);
  const bool mixed = k_head_bits != nullptr || v_head_bits != nullptr;
  if (mixed && Hkv > pqkv::kMaxListHeads)
    return fail(PQKV_ERR_UNSUPPORTED, "prefill: mixed widths support at most %d kv heads", pqkv::kMaxListHeads);
  if (!supported_bits(k_bits) && !k_head_bits) return fail(PQKV_ERR_UNSUPPORTED, "prefill: k_bits=%d", k_bits);
  if (!supported_bits(v_bits) && !v_head_bits) return fail(PQKV_ERR_UNSUPPORTED, "prefill: v_bits=%d", v_bits);
  int kb[pqkv::kMaxListHeads], vb[pqkv::kMaxListHeads];
  if (mixed)
    for (int h = 0; h < Hkv; ++h) {
      kb[h] = k_head_bits ? k_head_bits[h] : k_bits;
      vb[h] = v_head_bits ? v_head_bits[h] : v_bits;
      if (!supported_bits(kb[h]) || !supported_bits(vb[h]))
        return fail(PQKV_ERR_UNSUPPORTED, "prefill: head %d widths k=%d v=%d", h, kb[h], vb[h]);
    }
  if (qjl != (p_rot != nullptr)) return fail(PQKV_ERR_INVALID, "prefill: qjl and p_rot go together");
  if (pg && (mixed || k_bits != v_bits))
    return fail(PQKV_ERR_UNSUPPORTED, "prefill: paged caches take uniform widths with k_bits == v_bits");
  if (qjl && m != d) return fail(PQKV_ERR_UNSUPPORTED, "prefill: QJL needs m == d");
  if (!float_dtype(q_dtype) || !float_dtype(out_dtype)) return fail(PQKV_ERR_UNSUPPORTED, "prefill: dtype");
  if (!(scale > 0.0f) || !std::isfinite(scale)) return fail(PQKV_ERR_INVALID, "prefill: scale must be > 0");
  if (Sq == 0) return PQKV_OK;
  if (!q || !R || !out) return fail(PQKV_ERR_INVALID, "prefill: null pointer");
  if ((uintptr_t)R % 16) return fail(PQKV_ERR_INVALID, "prefill: R must be 16-byte aligned");
  if ((uintptr_t)p_rot % 16) return fail(PQKV_ERR_INVALID, "prefill: p_rot must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  if (S == 0) {
    const size_t ob = (size_t)B * Hq * Sq * d * (out_dtype == PQKV_F32 ? 4 : 2);
    return hip_status(pqkv::launch_fill_zero(out, ob, st), "prefill zero fill");
  }
  if ((pg ? (!pg->k_pages || !pg->v_pages) : (!k_cache || !v_cache)) || !k_codebooks || !v_codebooks)
    return fail(PQKV_ERR_INVALID, "prefill: null cache or codebook");
  const size_t need = pqkv_prefill_workspace_bytes(B, Hq, Hkv, Sq, S, d);
  if (!workspace || workspace_bytes < need)
    return fail(PQKV_ERR_WORKSPACE, "prefill: workspace %zu < %zu bytes", workspace_bytes, need);
  const int64_t nvec = (int64_t)B * Hq * Sq;
  const size_t arr = align256((size_t)nvec * d * 4);
  float *q32 = (float *)workspace;
  float *o32 = (float *)((char *)workspace + arr);
  float *pq32 = (float *)((char *)workspace + 2 * arr);
  const float kLog2e = 1.4426950408889634f;
  int tok = pqkv::prof_begin("prefill_rotate", st);
  // the kernel's queries carry kPrefillPlaneScale; the projections do not
  const float qs = scale * kLog2e * pqkv::kPrefillPlaneScale;
  hipError_t e = qjl ? pqkv::launch_rotate2(q, q_dtype, R, p_rot, q32, pq32, nvec, d, qs,
                                            1.0f / ((float)m * pqkv::kPrefillPlaneScale), st)
                     : pqkv::launch_rotate(q, q_dtype, R, q32, PQKV_F32, nvec, d, 0, qs, st);
  pqkv::prof_end(tok, st);
  if (e != hipSuccess) return hip_status(e, "prefill query rotation");
  pqkv::PrefillArgs a;
  memset(&a, 0, sizeof(a));
  a.q = q32;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.k_cb = k_codebooks;
  a.v_cb = v_codebooks;
  a.cb_head_stride = mixed ? 16 : 0;
  a.qjl = qjl_signs;
  a.pq = qjl ? pq32 : nullptr;
  a.o = o32;
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.G = Hq / Hkv;
  a.Sq = Sq;
  a.q_start = q_start;
  a.S = S;
  a.S_max = S_max;
  a.d = d;
  a.causal = causal ? 1 : 0;
  a.qt = pqkv::prefill_rows_per_block(qjl) / a.G;
  if (pg) {
    a.k_pages = pg->k_pages;
    a.v_pages = pg->v_pages;
    a.s_pages = pg->s_pages;
    a.page_shift = pg->page_shift;
    a.max_pages = pg->max_pages;
  }
  if (!mixed) {
    a.k_head_stride = (int64_t)S_max * pqkv_vector_bytes(d, k_bits);
    a.v_head_stride = (int64_t)S_max * pqkv_vector_bytes(d, v_bits);
    a.k_batch_stride = a.k_head_stride * Hkv;
    a.v_batch_stride = a.v_head_stride * Hkv;
    a.n_heads = Hkv;
    tok = pqkv::prof_begin("prefill_attn", st, true);
    e = hipSuccess;
    for (int rep = 0, nrep = pqkv::prof_repeats(); rep < nrep && e == hipSuccess; ++rep)
      e = pqkv::launch_prefill(a, k_bits, v_bits, st);
    pqkv::prof_end(tok, st);
    if (e != hipSuccess) return hip_status(e, "prefill launch");
  } else {
    // per-(b, h) runs of S_max vectors of the head's own width, (b, h) order;
    // one launch per (key bits, value bits) group of heads
    int64_t koff[pqkv::kMaxListHeads + 1], voff[pqkv::kMaxListHeads + 1];
    koff[0] = voff[0] = 0;
    for (int h = 0; h < Hkv; ++h) {
      koff[h + 1] = koff[h] + (int64_t)S_max * pqkv_vector_bytes(d, kb[h]);
      voff[h + 1] = voff[h] + (int64_t)S_max * pqkv_vector_bytes(d, vb[h]);
    }
    a.k_batch_stride = koff[Hkv];
    a.v_batch_stride = voff[Hkv];
    a.listed = 1;
    for (int kbits : {4, 2})
      for (int vbits : {4, 2}) {
        int n = 0;
        for (int h = 0; h < Hkv; ++h)
          if (kb[h] == kbits && vb[h] == vbits) {
            a.heads[n] = (int16_t)h;
            a.k_head_off[n] = koff[h];
            a.v_head_off[n] = voff[h];
            ++n;
          }
        if (n == 0) continue;
        a.n_heads = n;
        tok = pqkv::prof_begin("prefill_attn", st, true);
        e = hipSuccess;
        for (int rep = 0, nrep = pqkv::prof_repeats(); rep < nrep && e == hipSuccess; ++rep)
          e = pqkv::launch_prefill(a, kbits, vbits, st);
        pqkv::prof_end(tok, st);
        if (e != hipSuccess) return hip_status(e, "prefill launch");
      }
  }
  tok = pqkv::prof_begin("prefill_out_rotate", st);
  e = pqkv::launch_rotate(o32, PQKV_F32, R, out, out_dtype, nvec, d, 1, 1.0f, st);
  pqkv::prof_end(tok, st);
  return hip_status(e, "prefill output rotation");
}

}  // namespace pqkv

// ---- paged caches ----

namespace {

// log2 of a page size that is a power of two in [64, 65536], else -1
int page_shift_of(int page_tokens) {
  if (page_tokens < 64 || page_tokens > 65536 || (page_tokens & (page_tokens - 1))) return -1;
  int s = 0;
  while ((1 << s) < page_tokens) ++s;
  return s;
}

// Shared checks of the paged entry points: the page size, and a table wide
// enough for `positions` tokens per stream. Returns the page shift, or a
// negative status.
int paged_validate(const char *what, int page_tokens, int max_pages, int64_t positions) {
  const int shift = page_shift_of(page_tokens);
  if (shift < 0)
    return fail(PQKV_ERR_INVALID, "%s: page_tokens=%d is not a power of two in 64..65536", what, page_tokens);
  if (max_pages <= 0) return fail(PQKV_ERR_INVALID, "%s: max_pages=%d", what, max_pages);
  const int64_t need = (positions + page_tokens - 1) >> shift;
  if (need > max_pages)
    return fail(PQKV_ERR_INVALID, "%s: %lld positions need %lld pages per stream, the table has %d", what,
                (long long)positions, (long long)need, max_pages);
  return shift;
}

}  // namespace

extern "C" {

int pqkv_encode_paged(const void *x, int x_dtype, int64_t x_outer_stride, const float *R, const float *codebook,
                      int n_bits, uint8_t *const *pages, int page_tokens, int max_pages, int64_t start,
                      int64_t n_streams, int64_t n_tokens, int d, const float *p_rot, int m,
                      uint8_t *const *qjl_pages, void *stream) {
  if (start < 0) return fail(PQKV_ERR_INVALID, "encode_paged: start=%lld", (long long)start);
  if (n_streams < 0 || n_tokens < 0) return fail(PQKV_ERR_INVALID, "encode_paged: negative count");
  const int shift = paged_validate("encode_paged", page_tokens, max_pages, start + n_tokens);
  if (shift < 0) return shift;
  // the row checks of pqkv_encode with the page tables standing in for the
  // block and sign rows
  const int64_t vb = pqkv_vector_bytes(d, n_bits);
  const int v = encode_validate(x, x_dtype, x_outer_stride, R, codebook, n_bits, (uint8_t *)pages, n_tokens * vb,
                                n_streams, n_tokens, d, p_rot, m, (uint8_t *)qjl_pages, n_tokens * (m / 8));
  if (v <= 0) return v;
  pqkv::EncodeArgs a;
  memset(&a, 0, sizeof(a));
  a.x = x;
  a.x_outer_stride = x_outer_stride;
  a.R = R;
  a.codebook = codebook;
  a.bits = n_bits;
  a.n_outer = n_streams;
  a.n_inner = n_tokens;
  a.d = d;
  a.p_rot = p_rot;
  a.m = m;
  a.pages = pages;
  a.qjl_pages = qjl_pages;
  a.page_shift = shift;
  a.max_pages = max_pages;
  a.page_start = start;
  const char *env = getenv("PQKV_ENCODE_KERNEL");
  const bool exact = env && strcmp(env, "exact") == 0;
  hipError_t e;
  if (!exact && fast_encode_ok(x, x_dtype, x_outer_stride, n_streams, n_tokens, R, p_rot, (const uint8_t *)qjl_pages,
                                 0, nullptr, 0)) {
    const int tok = pqkv::prof_begin("encode_mfma", (hipStream_t)stream);
    e = pqkv::launch_encode_mfma(a, nullptr, nullptr, device_cus(), (hipStream_t)stream);
    pqkv::prof_end(tok, (hipStream_t)stream);
  } else {
    const int tok = pqkv::prof_begin("encode_exact", (hipStream_t)stream);
    e = pqkv::launch_encode_exact(a, x_dtype, (hipStream_t)stream);
    pqkv::prof_end(tok, (hipStream_t)stream);
  }
  return hip_status(e, "encode_paged launch");
}

int pqkv_decode_attn_paged(const void *q, int q_dtype, const float *R, const uint8_t *const *k_pages,
                           const uint8_t *const *v_pages, int page_tokens, int max_pages, const float *k_codebook,
                           const float *v_codebook, int n_bits, const uint8_t *const *qjl_pages, const float *p_rot,
                           int m, int B, int Hq, int Hkv, int S, int d, float scale, void *out, int out_dtype,
                           void *workspace, size_t workspace_bytes, void *stream) {
  const int shift = paged_validate("decode_paged", page_tokens, max_pages, S);
  if (shift < 0) return shift;
  const pqkv::PagedCache pg{k_pages, v_pages, qjl_pages, shift, max_pages};
  return pqkv::decode_attn_run(q, q_dtype, R, nullptr, nullptr, k_codebook, v_codebook, n_bits, n_bits, nullptr,
                               nullptr, nullptr, p_rot, m, B, Hq, Hkv, S, S, d, scale, out, out_dtype, workspace,
                               workspace_bytes, false, nullptr, stream, &pg);
}

int pqkv_prefill_attn_paged(const void *q, int q_dtype, const float *R, const uint8_t *const *k_pages,
                            const uint8_t *const *v_pages, int page_tokens, int max_pages, const float *k_codebook,
                            const float *v_codebook, int n_bits, const uint8_t *const *qjl_pages, const float *p_rot,
                            int m, int B, int Hq, int Hkv, int Sq, int q_start, int S, int d, float scale,
                            int causal, void *out, int out_dtype, void *workspace, size_t workspace_bytes,
                            void *stream) {
  const int shift = paged_validate("prefill_paged", page_tokens, max_pages, S);
  if (shift < 0) return shift;
  const pqkv::PagedCache pg{k_pages, v_pages, qjl_pages, shift, max_pages};
  return pqkv::prefill_attn_run(q, q_dtype, R, nullptr, nullptr, k_codebook, v_codebook, n_bits, n_bits, nullptr,
                                nullptr, nullptr, p_rot, m, B, Hq, Hkv, Sq, q_start, S, S, d, scale, causal, out,
                                out_dtype, workspace, workspace_bytes, stream, &pg);
}

int pqkv_dequantize(const uint8_t *blocks, const float *codebook, int n_bits, const float *R, void *out,
                    int out_dtype, int64_t n, int d, void *stream) {
  if (n < 0) return fail(PQKV_ERR_INVALID, "dequantize: n < 0");
  if (!supported_d(d) || !supported_bits(n_bits)) return fail(PQKV_ERR_UNSUPPORTED, "dequantize: d=%d bits=%d", d, n_bits);
  if (!float_dtype(out_dtype)) return fail(PQKV_ERR_UNSUPPORTED, "dequantize: dtype %d", out_dtype);
  if (n == 0) return PQKV_OK;
  if (!blocks || !codebook || !R || !out) return fail(PQKV_ERR_INVALID, "dequantize: null pointer");
  if ((uintptr_t)R % 16) return fail(PQKV_ERR_INVALID, "dequantize: R must be 16-byte aligned");
  const int tok = pqkv::prof_begin("dequantize", (hipStream_t)stream);
  const hipError_t e = pqkv::launch_dequantize(blocks, codebook, n_bits, R, out, out_dtype, n, d, (hipStream_t)stream);
  pqkv::prof_end(tok, (hipStream_t)stream);
  return hip_status(e, "dequantize launch");
}

int pqkv_soa_to_blocks(const uint8_t *packed, const float *radius, uint8_t *blocks, int64_t n, int d,
                       void *stream) {
  if (n < 0) return fail(PQKV_ERR_INVALID, "soa_to_blocks: n < 0");
  if (!supported_d(d)) return fail(PQKV_ERR_UNSUPPORTED, "soa_to_blocks: d=%d", d);
  if (n == 0) return PQKV_OK;
  if (!packed || !radius || !blocks) return fail(PQKV_ERR_INVALID, "soa_to_blocks: null pointer");
  return hip_status(pqkv::launch_soa_to_blocks(packed, radius, blocks, n, d, (hipStream_t)stream),
                    "soa_to_blocks launch");
}

int pqkv_blocks_to_soa(const uint8_t *blocks, uint8_t *packed, float *radius, int64_t n, int d, void *stream) {
  if (n < 0) return fail(PQKV_ERR_INVALID, "blocks_to_soa: n < 0");
  if (!supported_d(d)) return fail(PQKV_ERR_UNSUPPORTED, "blocks_to_soa: d=%d", d);
  if (n == 0) return PQKV_OK;
  if (!packed || !radius || !blocks) return fail(PQKV_ERR_INVALID, "blocks_to_soa: null pointer");
  return hip_status(pqkv::launch_blocks_to_soa(blocks, packed, radius, n, d, (hipStream_t)stream),
                    "blocks_to_soa launch");
}

}  // extern "C"
