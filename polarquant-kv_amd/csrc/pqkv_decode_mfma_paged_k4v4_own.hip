// Decode kernel instantiations for paged caches: 4-bit keys and values, values with a codebook of their own.
#include "pqkv_decode_mfma.h"

namespace pqkv {

hipError_t launch_dm_paged_k4v4_own(const DecodeArgs &a, hipStream_t s) {
  return launch_dm_widths<4, 4, false, true>(a, s);
}

}  // namespace pqkv
