// Decode launch dispatch: picks the translation unit of the width pair.
#include "pqkv_decode_mfma.h"

namespace pqkv {

hipError_t launch_decode_mfma(const DecodeArgs &a, int k_bits, int v_bits, hipStream_t s) {
  if (k_bits == 4 && v_bits == 4)
    return a.k_cb == a.v_cb ? launch_dm_k4v4_shared(a, s) : launch_dm_k4v4_own(a, s);  // one codebook: one table
  if (k_bits == 4) return launch_dm_k4v2(a, s);
  if (v_bits == 4) return launch_dm_k2v4(a, s);
  return launch_dm_k2v2(a, s);
}

hipError_t launch_decode_mfma_paged(const DecodeArgs &a, int bits, hipStream_t s) {
  if (bits == 4) return a.k_cb == a.v_cb ? launch_dm_paged_k4v4_shared(a, s) : launch_dm_paged_k4v4_own(a, s);
  return launch_dm_paged_k2v2(a, s);
}

}  // namespace pqkv
