// Activation arithmetic shared by the elementwise kernels and the GEMM
// epilogues that fuse them, so a fused and an unfused evaluation round
// identically.
#pragma once

#include <hip/hip_runtime.h>

namespace cnhip {

// ReLU forward, max(0, x) (relu.cpp:97-160); one expression for the
// elementwise kernel and every fused epilogue, so they agree on signed zeros.
__device__ __forceinline__ float relu_f(float x) { return fmaxf(0.f, x); }

// ReLU backward mask from the cached OUTPUT (relu_grad.cu:11-19): dy * [y > 0]
__device__ __forceinline__ float relu_mask(float y) { return y > 0.f ? 1.f : 0.f; }

// GELU, exact form x Phi(x) with Phi(x) = 0.5 erfc(-x/sqrt 2): the erfc form
// keeps full relative accuracy in the negative tail, where 1 + erf(.) cancels.
__device__ __forceinline__ float gelu_f(float v) {
  return v * (0.5f * erfcf(v * -0.70710678118654752440f));
}
// d GELU / dx = Phi(x) + x phi(x)
__device__ __forceinline__ float gelu_grad_f(float v) {
  const float cdf = 0.5f * erfcf(v * -0.70710678118654752440f);
  const float pdf = 0.39894228040143267794f * expf(-0.5f * v * v);
  return cdf + v * pdf;
}

}  // namespace cnhip
