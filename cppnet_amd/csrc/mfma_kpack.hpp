// fp32 MFMA tile engine (v_mfma_f32_32x32x2f32, wave64), used by the GEMM
// and the Conv2D kernels.
//
// A block of WGM x WGN (x WGK) wavefronts owns a BM x BN output tile, BM =
// WGM*WM*32, BN = WGN*WN*32; each wave holds WM x WN accumulator blocks of
// 32x32 (16 floats per lane each).  K advances KT = BK*WGK at a time: with
// WGK > 1 the WGK wave groups each take a BK-deep slice of every k-tile
// (for tiles with few outputs and a long contraction) and their accumulators
// are summed at the end in a fixed order (reduce_wgk).
//
// Which k a lane feeds to which MFMA step is free, as long as A and B agree:
// in step t (t = 0 .. BK/2-1) lane half h = lane/32 supplies k = h*BK/2 + t,
// so a lane needs 4 consecutive k of one row per 4 steps (a "fragment").
//
// Each operand tile keeps the orientation it has in memory (Operand below):
// rows that are k-contiguous in memory are stored [rows][k] and a fragment
// is one ds_read_b128; rows contiguous along the output dimension are stored
// [k][rows] and a fragment is four ds_read_b32 at the same row.  Either way
// global -> LDS moves 16-byte float4s with conflict-free ds_write_b128, with
// no register transposes, and the fragment reads of the two half-waves fall
// into disjoint bank halves.  Staging goes through registers (two k-tiles in
// flight, double-buffered LDS, one barrier per k-tile: pipeline below), and
// every thread does the same work, so the compiler counts outstanding loads
// exactly.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace cnhip {
namespace kp {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int WGM_, int WGN_, int WM_, int WN_, int BK_ = 16, int WGK_ = 1>
struct Cfg {
  static constexpr int WGM = WGM_, WGN = WGN_, WM = WM_, WN = WN_;
  static constexpr int BK = BK_, WGK = WGK_;
  static constexpr int KT = BK * WGK;  // k-tile depth
  static constexpr int BM = WGM * WM * 32;
  static constexpr int BN = WGN * WN * 32;
  static constexpr int NT = WGM * WGN * WGK * 64;
  static_assert(BK == 16 || BK == 32, "BK must be 16 or 32");
  static_assert(WGK == 1 || WGK == 2 || WGK == 4 || WGK == 8, "WGK must be 1, 2, 4 or 8");
};

// Wave -> (wm, wn, wk) position in the block.
template <class C>
__device__ __forceinline__ void wave_pos(int& wm, int& wn, int& wk) {
  const int wave = threadIdx.x >> 6;
  wm = wave % C::WGM;
  wn = C::WGK > 1 ? (wave / C::WGM) % C::WGN : wave / C::WGM;
  wk = C::WGK > 1 ? wave / (C::WGM * C::WGN) : 0;
}

// An R x KT operand tile in LDS.
//   KC:  X(r, k) = X[k + ld*r], rows k-contiguous.  LDS [R][KT+4]; a unit is
//        the 16-byte chunk X(r, k..k+3), one float4 load along k.
//   !KC: X(r, k) = X[r + ld*k], rows contiguous along r.  LDS [KT][R+4]; a
//        unit is X(r..r+3, k), one float4 load along r.
// Consecutive lanes take consecutive units, so global loads are coalesced
// and the ds_write_b128s hit consecutive (KC: padded) 16-byte slots.  The
// +4 padding makes the fragment reads conflict-free: KC, the b128 reads of 8
// consecutive lanes start 8 distinct 4-bank groups apart; !KC, the two
// half-waves read rows BK/2 k-rows apart, 32 banks apart for BK = 16.
template <bool KC, int R, int NT, int KT>
struct Operand {
  static constexpr int LD = KC ? KT + 4 : R + 4;        // LDS row stride (floats)
  static constexpr int FLOATS = KC ? R * LD : KT * LD;  // one tile
  static constexpr int CH = KC ? KT / 4 : R / 4;        // units per LDS row
  static constexpr int UNITS = R * KT / 4;
  static constexpr int PER = (UNITS + NT - 1) / NT;
  static constexpr int REGS = PER;

  // Unit p of this thread: KC, row r and k..k+3; !KC, rows r..r+3 and k.
  __device__ __forceinline__ static bool origin(int p, int& r, int& k) {
    const int u = threadIdx.x + NT * p;
    if (UNITS % NT != 0 && u >= UNITS) return false;
    if (KC) {
      r = u / CH;
      k = (u % CH) * 4;
    } else {
      k = u / CH;
      r = (u % CH) * 4;
    }
    return true;
  }

  // FAST: the whole tile is in range and 16-byte aligned.  Otherwise every
  // element is bounds-checked (rows < Rtot, k < Kend) and zero-filled.
  template <bool FAST>
  __device__ __forceinline__ static void load(const float* __restrict__ X, int64_t ld, int64_t r0,
                                              int64_t k0, int64_t Rtot, int64_t Kend,
                                              f32x4 (&v)[REGS]) {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      int r, k;
      if (!origin(p, r, k)) break;
      const int64_t gr = r0 + r, gk = k0 + k;
      if (FAST) {
        v[p] = *reinterpret_cast<const f32x4*>(X + (KC ? gk + ld * gr : gr + ld * gk));
      } else {
        f32x4 t;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const bool in = KC ? (gr < Rtot && gk + j < Kend) : (gr + j < Rtot && gk < Kend);
          t[j] = in ? X[KC ? gk + j + ld * gr : gr + j + ld * gk] : 0.f;
        }
        v[p] = t;
      }
    }
  }

  __device__ __forceinline__ static void store(float* __restrict__ lds, const f32x4 (&v)[REGS]) {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      int r, k;
      if (!origin(p, r, k)) break;
      *reinterpret_cast<f32x4*>(lds + (KC ? r * LD + k : k * LD + r)) = v[p];
    }
  }

  // Fragment X(row, k..k+3) from the LDS tile.
  __device__ __forceinline__ static f32x4 frag(const float* __restrict__ lds, int row, int k) {
    if (KC) return *reinterpret_cast<const f32x4*>(lds + row * LD + k);
    const float* q = lds + k * LD + row;
    return f32x4{q[0], q[LD], q[2 * LD], q[3 * LD]};
  }
};

template <class C>
__device__ __forceinline__ void zero_acc(f32x16 (&acc)[C::WM][C::WN]) {
#pragma unroll
  for (int i = 0; i < C::WM; ++i)
#pragma unroll
    for (int j = 0; j < C::WN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
}

// One k-tile of the block's MFMA work from the LDS tiles la (operand OA)
// and lb (operand OB): each wave runs the BK-deep slice wk of it; chunk c,
// element e is step t = 4c + e.
template <class C, class OA, class OB>
__device__ __forceinline__ void mfma_ktile(const float* __restrict__ la,
                                           const float* __restrict__ lb,
                                           f32x16 (&acc)[C::WM][C::WN]) {
  const int lane = threadIdx.x & 63;
  int wm, wn, wk;
  wave_pos<C>(wm, wn, wk);
  const int h = lane >> 5, r = lane & 31;
  const int ra = wm * (C::WM * 32) + r, rb = wn * (C::WN * 32) + r;
  const int kb = wk * C::BK + (C::BK / 2) * h;
  // Waves with 2 x 2 or more accumulator blocks raise their issue priority
  // for the k-tile's MFMAs, so a SIMD's matrix pipe is fed ahead of the other
  // waves' staging loads (config 2's 128 x 256 tiles: 0.9% per train step,
  // measured; the 128 x 128 tile was measured slower with it).
  if constexpr (C::WM * C::WN >= 4) __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int c = 0; c < C::BK / 8; ++c) {
    f32x4 a[C::WM], b[C::WN];
#pragma unroll
    for (int i = 0; i < C::WM; ++i) a[i] = OA::frag(la, ra + 32 * i, kb + 4 * c);
#pragma unroll
    for (int j = 0; j < C::WN; ++j) b[j] = OB::frag(lb, rb + 32 * j, kb + 4 * c);
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int i = 0; i < C::WM; ++i)
#pragma unroll
        for (int j = 0; j < C::WN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][e], b[j][e], acc[i][j], 0, 0, 0);
  }
  if constexpr (C::WM * C::WN >= 4) __builtin_amdgcn_s_setprio(0);
}

// Visits the accumulators: f(m_local, n_local, 4 values at rows m..m+3).
// Accumulator layout of v_mfma_f32_32x32x2f32: lane holds column n = lane%32
// and rows 8*(r/4) + 4*(lane/32) + r%4, r = 0..15.
// With WGK > 1 only the wk == 0 waves (which hold the reduce_wgk sums) visit.
template <class C, class F>
__device__ __forceinline__ void for_each_acc_run(const f32x16 (&acc)[C::WM][C::WN], F&& f) {
  const int lane = threadIdx.x & 63;
  int wm, wn, wk;
  wave_pos<C>(wm, wn, wk);
  if (C::WGK > 1 && wk != 0) return;
#pragma unroll
  for (int i = 0; i < C::WM; ++i)
#pragma unroll
    for (int j = 0; j < C::WN; ++j) {
      const int n = wn * (C::WN * 32) + j * 32 + (lane & 31);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = wm * (C::WM * 32) + i * 32 + 8 * q + 4 * (lane >> 5);
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[i][j][4 * q + e];
        f(m, n, v);
      }
    }
}

// Sums the accumulators of the WGK wave groups into the wk == 0 waves, in
// the order wk = 0, 1, .., WGK-1, through LDS (lds: at least
// (WGK-1) * WGM*WGN * WM*WN * 16 * 64 floats, free for reuse: the caller's
// last barrier has passed).  No-op for WGK == 1.
template <class C>
__device__ __forceinline__ void reduce_wgk(float* lds, f32x16 (&acc)[C::WM][C::WN]) {
  if constexpr (C::WGK > 1) {
    const int lane = threadIdx.x & 63;
    int wm, wn, wk;
    wave_pos<C>(wm, wn, wk);
    constexpr int PER_WAVE = C::WM * C::WN * 16 * 64;
    const int slot = wm + C::WGM * wn;
    if (wk > 0) {
      float* dst = lds + ((wk - 1) * C::WGM * C::WGN + slot) * PER_WAVE;
#pragma unroll
      for (int i = 0; i < C::WM; ++i)
#pragma unroll
        for (int j = 0; j < C::WN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) dst[((i * C::WN + j) * 16 + r) * 64 + lane] = acc[i][j][r];
    }
    __syncthreads();
    if (wk == 0) {
#pragma unroll
      for (int g = 1; g < C::WGK; ++g) {
        const float* src = lds + ((g - 1) * C::WGM * C::WGN + slot) * PER_WAVE;
#pragma unroll
        for (int i = 0; i < C::WM; ++i)
#pragma unroll
          for (int j = 0; j < C::WN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] += src[((i * C::WN + j) * 16 + r) * 64 + lane];
      }
    }
  }
}

// ------------------------------------------------------------------
// 16 x 16 accumulator tiles (v_mfma_f32_16x16x4f32), for problems whose
// output is too small to give every CU a 32 x 32 tile.  Same Operand tiles
// and pipeline; a wave holds WM x WN blocks of 16 x 16 (4 floats per lane).
// In each 4-step group, lane group q = lane/16 supplies k = 4q + step, so a
// lane's fragment is again 4 consecutive k of one row (one ds_read_b128 for
// k-contiguous tiles, four ds_read_b32 otherwise; the four lane groups sit
// 16 banks apart in both layouts).
template <int WGM_, int WGN_, int WM_, int WN_, int BK_ = 16, int WGK_ = 1>
struct Cfg16 {
  static constexpr int WGM = WGM_, WGN = WGN_, WM = WM_, WN = WN_;
  static constexpr int BK = BK_, WGK = WGK_;
  static constexpr int KT = BK * WGK;
  static constexpr int BM = WGM * WM * 16;
  static constexpr int BN = WGN * WN * 16;
  static constexpr int NT = WGM * WGN * WGK * 64;
  static_assert(BK % 16 == 0, "BK must be a multiple of 16");
  static_assert(WGK == 1 || WGK == 2 || WGK == 4 || WGK == 8, "WGK must be 1, 2, 4 or 8");
};

template <class C>
__device__ __forceinline__ void zero_acc16(f32x4 (&acc)[C::WM][C::WN]) {
#pragma unroll
  for (int i = 0; i < C::WM; ++i)
#pragma unroll
    for (int j = 0; j < C::WN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
}

template <class C, class OA, class OB>
__device__ __forceinline__ void mfma_ktile16(const float* __restrict__ la,
                                             const float* __restrict__ lb,
                                             f32x4 (&acc)[C::WM][C::WN]) {
  const int lane = threadIdx.x & 63;
  int wm, wn, wk;
  wave_pos<C>(wm, wn, wk);
  const int q = lane >> 4, r = lane & 15;
  const int ra = wm * (C::WM * 16) + r, rb = wn * (C::WN * 16) + r;
  const int kb = wk * C::BK + 4 * q;
#pragma unroll
  for (int c = 0; c < C::BK / 16; ++c) {
    f32x4 a[C::WM], b[C::WN];
#pragma unroll
    for (int i = 0; i < C::WM; ++i) a[i] = OA::frag(la, ra + 16 * i, kb + 16 * c);
#pragma unroll
    for (int j = 0; j < C::WN; ++j) b[j] = OB::frag(lb, rb + 16 * j, kb + 16 * c);
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int i = 0; i < C::WM; ++i)
#pragma unroll
        for (int j = 0; j < C::WN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][e], b[j][e], acc[i][j], 0, 0, 0);
  }
}

// Accumulator layout of v_mfma_f32_16x16x4f32: lane holds column lane%16
// and rows 4*(lane/16) + r, r = 0..3.  Only wk == 0 waves visit.
template <class C, class F>
__device__ __forceinline__ void for_each_acc_run16(const f32x4 (&acc)[C::WM][C::WN], F&& f) {
  const int lane = threadIdx.x & 63;
  int wm, wn, wk;
  wave_pos<C>(wm, wn, wk);
  if (C::WGK > 1 && wk != 0) return;
#pragma unroll
  for (int i = 0; i < C::WM; ++i)
#pragma unroll
    for (int j = 0; j < C::WN; ++j)
      f(wm * (C::WM * 16) + i * 16 + 4 * (lane >> 4), wn * (C::WN * 16) + j * 16 + (lane & 15),
        acc[i][j]);
}

// reduce_wgk for 16 x 16 accumulators: (WGK-1) * WGM*WGN * WM*WN * 4 * 64
// floats of lds.
template <class C>
__device__ __forceinline__ void reduce_wgk16(float* lds, f32x4 (&acc)[C::WM][C::WN]) {
  if constexpr (C::WGK > 1) {
    const int lane = threadIdx.x & 63;
    int wm, wn, wk;
    wave_pos<C>(wm, wn, wk);
    constexpr int PER_WAVE = C::WM * C::WN * 4 * 64;
    const int slot = wm + C::WGM * wn;
    if (wk > 0) {
      float* dst = lds + ((wk - 1) * C::WGM * C::WGN + slot) * PER_WAVE;
#pragma unroll
      for (int i = 0; i < C::WM; ++i)
#pragma unroll
        for (int j = 0; j < C::WN; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) dst[((i * C::WN + j) * 4 + r) * 64 + lane] = acc[i][j][r];
    }
    __syncthreads();
    if (wk == 0) {
#pragma unroll
      for (int g = 1; g < C::WGK; ++g) {
        const float* src = lds + ((g - 1) * C::WGM * C::WGN + slot) * PER_WAVE;
#pragma unroll
        for (int i = 0; i < C::WM; ++i)
#pragma unroll
          for (int j = 0; j < C::WN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][r] += src[((i * C::WN + j) * 4 + r) * 64 + lane];
      }
    }
  }
}

// LDS floats of one pipeline buffer of a stage (A tile, then B tile); the
// pipeline double-buffers it.
template <class Stage>
constexpr int stage_floats() {
  return Stage::OA::FLOATS + Stage::OB::FLOATS;
}

// Software pipeline over ntiles k-tiles: tile t+1 and t+2 are in flight in
// two register sets while tile t is multiplied from LDS (double-buffered, one
// barrier per k-tile).  The stage names its operands OA and OB and supplies
// load<S>(t) (global -> register set S) and store<S>(buf) (register set S ->
// an LDS buffer: A tile, then B tile at OA::FLOATS); the loop is unrolled by
// two so the sets alternate statically.  lds holds 2 * stage_floats<Stage>().
// The loop body runs whole tile pairs and has no exit in its middle, and an
// odd last tile is done after it: with a single exit the accumulators keep
// one register assignment around the loop (a mid-body exit made the compiler
// copy every accumulator between two register sets each iteration).
// Ends with a barrier, after which lds may be reused.
template <class C, class OA, class OB, class Acc>
__device__ __forceinline__ void ktile_any(const float* la, const float* lb, Acc& acc) {
  if constexpr (sizeof(acc[0][0]) == sizeof(f32x16))
    mfma_ktile<C, OA, OB>(la, lb, acc);
  else
    mfma_ktile16<C, OA, OB>(la, lb, acc);
}

template <class C, class Stage, class Acc>
__device__ __forceinline__ void pipeline(int ntiles, float* lds, Stage& s, Acc& acc) {
  using OA = typename Stage::OA;
  using OB = typename Stage::OB;
  float* buf0 = lds;
  float* buf1 = lds + stage_floats<Stage>();
  constexpr int BOFF = OA::FLOATS;
  if (ntiles > 0) {
    s.template load<0>(0);
    s.template store<0>(buf0);
  }
  if (ntiles > 1) s.template load<0>(1);
  if (ntiles > 2) s.template load<1>(2);
  __syncthreads();
  int kt = 0;
  for (; kt + 1 < ntiles; kt += 2) {
    // tile kt in buf0, kt+1 in set 0, kt+2 in set 1
    ktile_any<C, OA, OB>(buf0, buf0 + BOFF, acc);
    s.template store<0>(buf1);
    if (kt + 3 < ntiles) s.template load<0>(kt + 3);
    __syncthreads();
    // tile kt+1 in buf1, kt+2 in set 1, kt+3 in set 0
    ktile_any<C, OA, OB>(buf1, buf1 + BOFF, acc);
    if (kt + 2 < ntiles) {
      s.template store<1>(buf0);
      if (kt + 4 < ntiles) s.template load<1>(kt + 4);
    }
    __syncthreads();
  }
  if (kt < ntiles) {  // odd count: the last tile is in buf0
    ktile_any<C, OA, OB>(buf0, buf0 + BOFF, acc);
    __syncthreads();
  }
}

}  // namespace kp
}  // namespace cnhip
