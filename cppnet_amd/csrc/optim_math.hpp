// Optimizer arithmetic shared by the optimizer kernels (adam.hip) and the
// fused train-step kernels (mlp_step.hip), so both round identically.
#pragma once

#include <hip/hip_runtime.h>

namespace cnhip {

struct AdamHyper {
  float lr, b1, b2, eps;
};

// One Adam element update (adam.cpp:98-133), evaluated without contraction
// in the reference's order: m, v, the bias-corrected moments, the step.
__device__ __forceinline__ void adam_one(float& w, float g, float& m, float& v, float bc1,
                                         float bc2, const AdamHyper& h) {
#pragma clang fp contract(off)
  m = h.b1 * m + (1.0f - h.b1) * g;
  v = h.b2 * v + (1.0f - h.b2) * g * g;
  const float mh = m / bc1;
  const float vh = v / bc2;
  w -= h.lr * mh / (sqrtf(vh) + h.eps);
}

}  // namespace cnhip
