// Allocation-free decode entry point: pqkv_decode_attn with its workspace
// (rotated queries, split partials, QJL projections) taken from a
// file-scope device array instead of a caller buffer, for callers that
// cannot allocate device memory (code under stream or graph capture, tight
// serving loops). The array is part of the library's code object, so every
// GPU the library runs on holds its own copy, at its own address, until the
// process ends.
//
// Host code never uses the array's name as an address: the name is a host
// stand-in. The device address comes from hipGetSymbolAddress, once per
// device with that device current, and only that address reaches kernels.
//
// Every call on one GPU shares that GPU's array. Nothing in it needs to start
// at zero (each byte a call reads was written earlier in the same call), but
// two calls that overlap in time on one GPU (different streams, or host
// threads without ordering) race on it.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/pqkv.h"
#include "pqkv_launch.h"

static __device__ __align__(256) uint8_t scratch[PQKV_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// Device address of this device's scratch array (resolved on the first call
// made with the device current); nullptr with *err set when it cannot be.
void *scratch_for_current_device(hipError_t *err) {
  int dev = -1;
  *err = hipGetDevice(&dev);
  if (*err != hipSuccess) return nullptr;
  if (dev < 0 || dev >= kMaxDevices) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void *p = nullptr;
    *err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (*err != hipSuccess || p == nullptr) {
      if (*err == hipSuccess) *err = hipErrorInvalidSymbol;
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" int pqkv_decode_attn_noalloc(const void *q, int q_dtype, const float *R, const uint8_t *k_cache,
                                        const uint8_t *v_cache, const float *k_codebooks,
                                        const float *v_codebooks, int k_bits, int v_bits, const int *k_head_bits,
                                        const int *v_head_bits, const uint8_t *qjl_signs, const float *p_rot,
                                        int m, int B, int Hq, int Hkv, int S, int S_max, int d, float scale,
                                        void *out, int out_dtype, void *stream) {
  hipError_t e = hipSuccess;
  void *ws = scratch_for_current_device(&e);
  if (ws == nullptr) return pqkv::report_hip_error(e, "decode_noalloc: scratch address");
  return pqkv::decode_attn_run(q, q_dtype, R, k_cache, v_cache, k_codebooks, v_codebooks, k_bits, v_bits,
                               k_head_bits, v_head_bits, qjl_signs, p_rot, m, B, Hq, Hkv, S, S_max, d, scale, out,
                               out_dtype, ws, (size_t)PQKV_NOALLOC_SCRATCH_BYTES, true, nullptr, stream);
}
