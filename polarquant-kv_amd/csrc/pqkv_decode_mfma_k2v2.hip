// Decode kernel instantiations: 2-bit keys, 2-bit values.
#include "pqkv_decode_mfma.h"

namespace pqkv {

hipError_t launch_dm_k2v2(const DecodeArgs &a, hipStream_t s) { return launch_dm_widths<2, 2>(a, s); }

}  // namespace pqkv
