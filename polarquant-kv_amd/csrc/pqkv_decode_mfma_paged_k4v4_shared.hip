// Decode kernel instantiations for paged caches: 4-bit keys and values, one shared codebook table.
#include "pqkv_decode_mfma.h"

namespace pqkv {

hipError_t launch_dm_paged_k4v4_shared(const DecodeArgs &a, hipStream_t s) {
  return launch_dm_widths<4, 4, true, true>(a, s);
}

}  // namespace pqkv
