// Decode kernel instantiations for the ggml flash-attn-ext layout: 4-bit keys
// and values with one codebook, tokens of a stream a stride apart, batch rows
// grouped into key / value sequences, fp16 additive mask.
#include "pqkv_decode_mfma.h"

namespace pqkv {

// kv heads in fours (n_heads % 4 == 0): one head per wave, so the waves of
// a workgroup read the same tokens' lines; otherwise the four waves share a
// head's chunks.
hipError_t launch_decode_mfma_ggml(const DecodeArgs &a, hipStream_t s) {
  const bool hw = ggml_heads_per_wave(a.n_heads);
  if (a.d == 128) {
    if (hw) launch_dm<128, 4, 4, false, true, false, true, true>(a, a.g, s);
    else launch_dm<128, 4, 4, false, true, false, true>(a, a.g, s);
  } else {
    if (hw) launch_dm<64, 4, 4, false, true, false, true, true>(a, a.g, s);
    else launch_dm<64, 4, 4, false, true, false, true>(a, a.g, s);
  }
  return hipGetLastError();
}

}  // namespace pqkv
