// Decode kernel instantiations: 2-bit keys, 4-bit values.
#include "pqkv_decode_mfma.h"

namespace pqkv {

hipError_t launch_dm_k2v4(const DecodeArgs &a, hipStream_t s) { return launch_dm_widths<2, 4>(a, s); }

}  // namespace pqkv
