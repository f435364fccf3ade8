// Mixed-width decode launches (4/4 and 2/2 kv heads in one grid).
#include "pqkv_decode_mfma.h"

namespace pqkv {

template <int D, bool QJL>
static void launch_dm_pair(const DecodeArgs &a4, const DecodeArgs &a2, int G, hipStream_t s) {
  dim3 grid(a4.splits, a4.B * a4.n_heads + a2.B * a2.n_heads);
  switch (G) {
    case 1: decode_mfma_pair_kernel<D, 1, QJL><<<grid, 256, 0, s>>>(a4, a2); break;
    case 2: decode_mfma_pair_kernel<D, 2, QJL><<<grid, 256, 0, s>>>(a4, a2); break;
    case 3: decode_mfma_pair_kernel<D, 3, QJL><<<grid, 256, 0, s>>>(a4, a2); break;
    case 4: decode_mfma_pair_kernel<D, 4, QJL><<<grid, 256, 0, s>>>(a4, a2); break;
    case 5: decode_mfma_pair_kernel<D, 5, QJL><<<grid, 256, 0, s>>>(a4, a2); break;
    case 6: decode_mfma_pair_kernel<D, 6, QJL><<<grid, 256, 0, s>>>(a4, a2); break;
    case 7: decode_mfma_pair_kernel<D, 7, QJL><<<grid, 256, 0, s>>>(a4, a2); break;
    default: decode_mfma_pair_kernel<D, 8, QJL><<<grid, 256, 0, s>>>(a4, a2); break;
  }
}

hipError_t launch_decode_mfma_pair(const DecodeArgs &a4, const DecodeArgs &a2, hipStream_t s) {
  const int G = a4.g;
  const bool qjl = a4.qjl != nullptr;
  if (a4.d == 128) {
    if (qjl) launch_dm_pair<128, true>(a4, a2, G, s);
    else launch_dm_pair<128, false>(a4, a2, G, s);
  } else {
    if (qjl) launch_dm_pair<64, true>(a4, a2, G, s);
    else launch_dm_pair<64, false>(a4, a2, G, s);
  }
  return hipGetLastError();
}


}  // namespace pqkv
