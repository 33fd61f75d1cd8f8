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

// exp(x) to about 1 ulp, branch-free: 2^(x log2 e) with x log2 e carried as
// a float y plus its rounding error (one fma and the low part of log2 e),
// the hardware exp2 (v_exp_f32, 1 ulp) applied to y and the error term
// folded in to first order.  Results below 2^-126 flush to zero.
__device__ __forceinline__ float exp_acc(float x) {
  constexpr float kLog2eHi = 1.44269502162933349609375f;  // log2(e) rounded to float
  constexpr float kLog2eLo = 1.9259629911e-8f;  // log2(e) - kLog2eHi
  constexpr float kLn2 = 0.693147180559945309417f;
  const float y = x * kLog2eHi;
  const float y_lo = fmaf(x, kLog2eLo, fmaf(x, kLog2eHi, -y));
  return __builtin_amdgcn_exp2f(y) * fmaf(y_lo, kLn2, 1.0f);
}

// erfc(z) for z >= 0 by the Chebyshev-fitted formula of Numerical Recipes
// (Press, Teukolsky, Vetterling and Flannery, 2nd ed., section 6.2, erfcc):
// erfc(z) = t exp(-z^2) exp(P(t)), t = 1 / (1 + z/2), P a degree-9
// polynomial, fractional error below 1.2e-7 in exact arithmetic for every
// z >= 0.  z^2 is split into its float value and exact remainder (one fma)
// so that exp(-z^2) keeps full precision; *e_z2 receives exp(-z^2) for the
// normal density.  Branch-free (the library erfcf takes one of several
// range branches per lane, and a wave pays for every branch its lanes
// take): config 5's GELU pass and its derivative in a GEMM epilogue are
// bound by this arithmetic.
__device__ __forceinline__ float erfc_nonneg(float z, float* e_z2) {
  const float t = __builtin_amdgcn_rcpf(fmaf(0.5f, z, 1.0f));
  float p = 0.17087277f;
  p = fmaf(t, p, -0.82215223f);
  p = fmaf(t, p, 1.48851587f);
  p = fmaf(t, p, -1.13520398f);
  p = fmaf(t, p, 0.27886807f);
  p = fmaf(t, p, -0.18628806f);
  p = fmaf(t, p, 0.09678418f);
  p = fmaf(t, p, 0.37409196f);
  p = fmaf(t, p, 1.00002368f);
  p = fmaf(t, p, -1.26551223f);
  const float s = z * z, s_lo = fmaf(z, z, -s);
  const float e = exp_acc(-s) * (1.0f - s_lo);
  *e_z2 = e;
  return (t * e) * exp_acc(p);
}

// Phi(v) = 0.5 erfc(-v / sqrt 2) from erfc of |v| / sqrt 2: 0.5 erfc(z) for
// v < 0 (full relative accuracy in the negative tail, where 1 + erf(.)
// would cancel), 1 - 0.5 erfc(z) for v >= 0.
__device__ __forceinline__ float ncdf_f(float v, float z, float* e_z2) {
  const float h = 0.5f * erfc_nonneg(z, e_z2);
  return v < 0.f ? h : 1.0f - h;
}

// GELU, exact form x Phi(x).
__device__ __forceinline__ float gelu_f(float v) {
  float e;
  return v * ncdf_f(v, fabsf(v) * 0.70710678118654752440f, &e);
}
// d GELU / dx = Phi(x) + x phi(x), phi(x) = exp(-x^2/2) / sqrt(2 pi)
__device__ __forceinline__ float gelu_grad_f(float v) {
  float e;  // exp(-z^2) = exp(-x^2/2)
  const float cdf = ncdf_f(v, fabsf(v) * 0.70710678118654752440f, &e);
  return fmaf(v, 0.39894228040143267794f * e, cdf);
}

}  // namespace cnhip
