// The sum of one column of a column-major matrix by one wave, in a fixed
// order: shared by the bias-gradient kernel (linear.hip) and the split-K
// reduce launch that also runs those sums (gemm_f32.hip), so both give the
// same bits.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace cnhip {

// Every lane returns the sum of p[0 .. rows): vec (rows % 4 == 0, p 16-byte
// aligned), four float4 loads in flight per lane into four running sums
// added in order; else lane-strided scalars; then a butterfly over the wave.
__device__ __forceinline__ float column_wave_sum(const float* __restrict__ p, int64_t rows, int vec, int lane) {
  typedef float f32x4_t __attribute__((ext_vector_type(4)));
  float s = 0.f;
  if (vec) {
    const int64_t n4 = rows >> 2;
    const f32x4_t* p4 = reinterpret_cast<const f32x4_t*>(p);
    f32x4_t a0 = {0.f, 0.f, 0.f, 0.f}, a1 = a0, a2 = a0, a3 = a0;
    int64_t i = lane;
    for (; i + 192 < n4; i += 256) {
      a0 += p4[i];
      a1 += p4[i + 64];
      a2 += p4[i + 128];
      a3 += p4[i + 192];
    }
    for (; i < n4; i += 64) a0 += p4[i];
    const f32x4_t t = (a0 + a1) + (a2 + a3);
    s = (t[0] + t[1]) + (t[2] + t[3]);
  } else {
    for (int64_t i = lane; i < rows; i += 64) s += p[i];
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  return s;
}

// Column sums of a column-major [rows, cols] matrix: out[c] (+)= sum of
// column c, one wave per column.
struct ColsumJob {
  const float* in;
  float* out;
  int64_t rows, cols;
  int accumulate, vec;
};

__device__ __forceinline__ void colsum_wave(const ColsumJob& cs, int64_t col, int lane) {
  if (col >= cs.cols) return;
  const float s = column_wave_sum(cs.in + cs.rows * col, cs.rows, cs.vec, lane);
  if (lane == 0) cs.out[col] = cs.accumulate ? cs.out[col] + s : s;
}

}  // namespace cnhip
