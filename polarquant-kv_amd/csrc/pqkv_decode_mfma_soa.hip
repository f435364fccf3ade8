// Decode over 4-bit caches in the reference kernels' SoA layout (packed
// codes + fp32 radii), for the reference-compatible entry points.
#include "pqkv_decode_mfma.h"

namespace pqkv {

hipError_t launch_decode_mfma_soa(const DecodeArgs &a, hipStream_t s) {
  const bool shared = a.k_cb == a.v_cb;
  if (a.d == 128) {
    if (shared) launch_dm<128, 4, 4, false, true, true>(a, a.g, s);
    else launch_dm<128, 4, 4, false, false, true>(a, a.g, s);
  } else {
    if (shared) launch_dm<64, 4, 4, false, true, true>(a, a.g, s);
    else launch_dm<64, 4, 4, false, false, true>(a, a.g, s);
  }
  return hipGetLastError();
}

}  // namespace pqkv
