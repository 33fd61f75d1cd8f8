// Shared fp32 MFMA tile engine (v_mfma_f32_32x32x2f32, wave64) used by the
// GEMM and the implicit-GEMM convolution kernels.
//
// A block of WGM x WGN wavefronts owns a BM x BN output tile, BM = WGM*WM*32,
// BN = WGN*WN*32; each wave holds WM x WN accumulator blocks of 32x32 (16
// floats per lane each).  K advances BK = 16 at a time: every thread stages
// float4s of the A and B tiles in registers, writes them to LDS as k-major
// rows (outer index contiguous, row stride +4 floats), and each wave then
// reads one ds_read_b32 per fragment: lane -> (r = lane%32, k = lane/32).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace cnhip {
namespace mfma {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int BK = 16;

template <int WGM_, int WGN_, int WM_, int WN_>
struct TileCfg {
  static constexpr int WGM = WGM_, WGN = WGN_, WM = WM_, WN = WN_;
  static constexpr int BM = WGM * WM * 32;
  static constexpr int BN = WGN * WN * 32;
  static constexpr int NT = WGM * WGN * 64;
  static constexpr int LDA = BM + 4;
  static constexpr int LDB = BN + 4;
};

// Thread -> (r, k) slot of a float4 in an R x BK operand tile.
//   KCONTIG: the float4 runs along k (4 consecutive k of one r);
//   otherwise it runs along r (4 consecutive r of one k).
template <bool KCONTIG, int R, int NT>
struct TileSlots {
  static constexpr int F4 = R * BK / 4;
  static constexpr int PER_THREAD = (F4 + NT - 1) / NT;
  __device__ __forceinline__ static bool slot(int p, int& rr, int& kk) {
    const int idx = threadIdx.x + NT * p;
    if (F4 % NT != 0 && idx >= F4) return false;
    if (KCONTIG) {
      rr = idx >> 2;
      kk = (idx & 3) * 4;
    } else {
      kk = idx / (R / 4);
      rr = (idx % (R / 4)) * 4;
    }
    return true;
  }
  // Writes staged float4s into LDS as [k][r] rows of stride R + 4.
  __device__ __forceinline__ static void store(float* __restrict__ lds,
                                               const f32x4 (&regs)[PER_THREAD]) {
    constexpr int LD = R + 4;
#pragma unroll
    for (int p = 0; p < PER_THREAD; ++p) {
      int rr, kk;
      if (!slot(p, rr, kk)) break;
      if (KCONTIG) {
#pragma unroll
        for (int j = 0; j < 4; ++j) lds[(kk + j) * LD + rr] = regs[p][j];
      } else {
        *reinterpret_cast<f32x4*>(lds + kk * LD + rr) = regs[p];
      }
    }
  }
};

template <class Cfg>
__device__ __forceinline__ void zero_acc(f32x16 (&acc)[Cfg::WM][Cfg::WN]) {
#pragma unroll
  for (int i = 0; i < Cfg::WM; ++i)
#pragma unroll
    for (int j = 0; j < Cfg::WN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
}

// One BK-deep step of the block's MFMA work from LDS tiles la/lb.
template <class Cfg>
__device__ __forceinline__ void mfma_ktile(const float* __restrict__ la,
                                           const float* __restrict__ lb,
                                           f32x16 (&acc)[Cfg::WM][Cfg::WN]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave % Cfg::WGM, wn = wave / Cfg::WGM;
  const float* pa = la + wm * (Cfg::WM * 32) + (lane & 31);
  const float* pb = lb + wn * (Cfg::WN * 32) + (lane & 31);
  const int lhi = lane >> 5;
#pragma unroll
  for (int s = 0; s < BK / 2; ++s) {
    const int k = 2 * s + lhi;
    float a[Cfg::WM], b[Cfg::WN];
#pragma unroll
    for (int i = 0; i < Cfg::WM; ++i) a[i] = pa[k * Cfg::LDA + 32 * i];
#pragma unroll
    for (int j = 0; j < Cfg::WN; ++j) b[j] = pb[k * Cfg::LDB + 32 * j];
#pragma unroll
    for (int i = 0; i < Cfg::WM; ++i)
#pragma unroll
      for (int j = 0; j < Cfg::WN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
  }
}

// Visits the accumulators: f(m_local, n_local, q, acc[i][j]) for the four
// runs of 4 consecutive rows each lane holds.  Accumulator layout of
// v_mfma_f32_32x32x2f32: lane holds column n = lane%32 and rows
// 8*(r/4) + 4*(lane/32) + r%4, r = 0..15.
template <class Cfg, class F>
__device__ __forceinline__ void for_each_acc_run(const f32x16 (&acc)[Cfg::WM][Cfg::WN], F&& f) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave % Cfg::WGM, wn = wave / Cfg::WGM;
#pragma unroll
  for (int i = 0; i < Cfg::WM; ++i)
#pragma unroll
    for (int j = 0; j < Cfg::WN; ++j) {
      const int n = wn * (Cfg::WN * 32) + j * 32 + (lane & 31);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = wm * (Cfg::WM * 32) + i * 32 + 8 * q + 4 * (lane >> 5);
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[i][j][4 * q + e];
        f(m, n, v);
      }
    }
}

}  // namespace mfma
}  // namespace cnhip
