// Decode kernel instantiations for paged caches: 2-bit keys, 2-bit values.
#include "pqkv_decode_mfma.h"

namespace pqkv {

hipError_t launch_dm_paged_k2v2(const DecodeArgs &a, hipStream_t s) {
  return launch_dm_widths<2, 2, false, true>(a, s);
}

}  // namespace pqkv
