// The fixed inputs of the ggml-side format, shared by the reference-
// compatible exports (pqkv_compat.cpp) and the GGML_TYPE_PQ4 type and ops
// (pqkv_ggml.cpp): the rotation generator and the codebook tables.
#pragma once

#include <cmath>
#include <cstdlib>

namespace pqkv {

// Orthogonal matrix from srand(seed)/rand() entries in [-1, 1] followed by
// row-wise Gram-Schmidt in float, the generator of polarquant_init
// (patch:549-579). Depends on the C library's rand().
inline void gram_schmidt_rotation(float *R, int D, unsigned seed) {
  srand(seed);
  for (int i = 0; i < D * D; ++i) {
    const float u = (float)rand() / (float)RAND_MAX;
    const float two_u = u * 2.0f;
    R[i] = two_u - 1.0f;
  }
  for (int i = 0; i < D; ++i) {
    for (int j = 0; j < i; ++j) {
      float dot = 0.0f;
      for (int k = 0; k < D; ++k) {
        const float p = R[i * D + k] * R[j * D + k];
        dot = dot + p;
      }
      for (int k = 0; k < D; ++k) {
        const float p = dot * R[j * D + k];
        R[i * D + k] = R[i * D + k] - p;
      }
    }
    float nrm = 0.0f;
    for (int k = 0; k < D; ++k) {
      const float p = R[i * D + k] * R[i * D + k];
      nrm = nrm + p;
    }
    nrm = sqrtf(nrm);
    if (nrm > 1e-10f)
      for (int k = 0; k < D; ++k) R[i * D + k] = R[i * D + k] / nrm;
  }
}

// The codebooks polarquant_init uploads, for every head_dim
// (patch:978-994, selected by n_bits at patch:600-613). They are a fixed
// input of the ggml format, so the values are the reference's, digit for
// digit.
inline constexpr float kGgmlCodebook4[16] = {-0.1547f, -0.1175f, -0.0928f, -0.0722f, -0.0537f, -0.0363f,
                                             -0.0193f, -0.0024f, 0.0145f,  0.0318f,  0.0498f,  0.0692f,
                                             0.0907f,  0.1157f,  0.1467f,  0.1947f};
inline constexpr float kGgmlCodebook3[8] = {-0.1350f, -0.0820f, -0.0440f, -0.0110f,
                                            0.0220f,  0.0560f,  0.0950f,  0.1500f};
inline constexpr float kGgmlCodebook2[4] = {-0.1050f, -0.0280f, 0.0400f, 0.1200f};

}  // namespace pqkv
