// fp32 MFMA tile engine with k-contiguous LDS operand tiles
// (v_mfma_f32_32x32x2f32, wave64), used by the GEMM kernel.
//
// A block of WGM x WGN (x WGK) wavefronts owns a BM x BN output tile, BM =
// WGM*WM*32, BN = WGN*WN*32; each wave holds WM x WN accumulator blocks of
// 32x32 (16 floats per lane each).  K advances KT = BK*WGK at a time: with
// WGK > 1 the WGK wave groups each take a BK-deep slice of every k-tile
// (for tiles with few outputs and a long contraction) and their accumulators
// are summed at the end in a fixed order (reduce_wgk).  Both operand tiles
// live in LDS as [rows][k] with k contiguous (row stride LDK = KT + 4 floats,
// so the 16-byte fragment reads of 8 consecutive lanes hit 8 distinct 4-bank
// groups).
//
// Which k a lane feeds to which MFMA step is free, as long as A and B agree:
// in step t (t = 0 .. BK/2-1) lane half h = lane/32 supplies k = h*BK/2 + t.
// A lane therefore needs BK/2 consecutive k of one row per operand block and
// fetches them with ds_read_b128s -- at BK = 16, 8 LDS reads feed the 32
// MFMAs of a 2 x 2 wave tile per k-tile.
//
// Global -> LDS staging goes through registers (double-buffered LDS, one
// barrier per k-tile).  An operand whose rows are k-contiguous in memory is
// moved as float4 along k; one whose rows are contiguous along the output
// dimension is gathered as four coalesced dwords per 16-byte LDS chunk.  Both
// write patterns are conflict-free, and every thread does the same work, so
// the compiler can count outstanding loads exactly.
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
  static constexpr int LDK = KT + 4;
  static constexpr int BM = WGM * WM * 32;
  static constexpr int BN = WGN * WN * 32;
  static constexpr int NT = WGM * WGN * WGK * 64;
  static constexpr int LDS_FLOATS = (BM + BN) * LDK;  // one buffer: A tile then B tile
  static_assert(BK == 16 || BK == 32, "BK must be 16 or 32");
  static_assert(WGK == 1 || WGK == 2 || WGK == 4, "WGK must be 1, 2 or 4");
};

// Wave -> (wm, wn, wk) position in the block.
template <class C>
__device__ __forceinline__ void wave_pos(int& wm, int& wn, int& wk) {
  const int wave = threadIdx.x >> 6;
  wm = wave % C::WGM;
  wn = C::WGK > 1 ? (wave / C::WGM) % C::WGN : wave / C::WGM;
  wk = C::WGK > 1 ? wave / (C::WGM * C::WGN) : 0;
}

// An R x BK operand tile.  KC: X(r, k) = X[k + ld*r] (k contiguous), else
// X(r, k) = X[r + ld*k] (r contiguous).  A unit is one 16-byte k-chunk of one
// row, written to LDS with one ds_write_b128.  KC loads it as one float4;
// otherwise as four dwords at consecutive k (consecutive lanes take
// consecutive rows, so each dword load is coalesced across the wave).
template <bool KC, int R, int NT, int BK>
struct Operand {
  static constexpr int LDK = BK + 4;
  static constexpr int CH = BK / 4;  // 16-byte chunks per row
  static constexpr int UNITS = R * CH;
  static constexpr int PER = (UNITS + NT - 1) / NT;
  static constexpr int REGS = PER;

  __device__ __forceinline__ static bool origin(int p, int& r, int& k) {
    const int u = threadIdx.x + NT * p;
    if (UNITS % NT != 0 && u >= UNITS) return false;
    if (KC) {  // chunk fastest: 8 consecutive lanes write 2 rows x 4 chunks
      r = u / CH;
      k = (u % CH) * 4;
    } else {  // row fastest: 8 consecutive lanes write 8 rows (80-float steps)
      r = u % R;
      k = (u / R) * 4;
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
      if (KC && FAST) {
        v[p] = *reinterpret_cast<const f32x4*>(X + gk + ld * gr);
      } else {
        f32x4 t;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t off = KC ? (gk + j + ld * gr) : (gr + ld * (gk + j));
          t[j] = (FAST || (gr < Rtot && gk + j < Kend)) ? X[off] : 0.f;
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
      *reinterpret_cast<f32x4*>(lds + r * LDK + k) = v[p];
    }
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

// One k-tile of the block's MFMA work from the LDS tiles la ([BM][LDK]) and
// lb ([BN][LDK]): each wave runs the BK-deep slice wk of it; chunk c,
// element e is step t = 4c + e.
template <class C>
__device__ __forceinline__ void mfma_ktile(const float* __restrict__ la,
                                           const float* __restrict__ lb,
                                           f32x16 (&acc)[C::WM][C::WN]) {
  const int lane = threadIdx.x & 63;
  int wm, wn, wk;
  wave_pos<C>(wm, wn, wk);
  const int h = lane >> 5, r = lane & 31;
  constexpr int LDK = C::LDK;
  const float* pa = la + (wm * (C::WM * 32) + r) * LDK + wk * C::BK + (C::BK / 2) * h;
  const float* pb = lb + (wn * (C::WN * 32) + r) * LDK + wk * C::BK + (C::BK / 2) * h;
#pragma unroll
  for (int c = 0; c < C::BK / 8; ++c) {
    f32x4 a[C::WM], b[C::WN];
#pragma unroll
    for (int i = 0; i < C::WM; ++i) a[i] = *reinterpret_cast<const f32x4*>(pa + i * 32 * LDK + 4 * c);
#pragma unroll
    for (int j = 0; j < C::WN; ++j) b[j] = *reinterpret_cast<const f32x4*>(pb + j * 32 * LDK + 4 * c);
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int i = 0; i < C::WM; ++i)
#pragma unroll
        for (int j = 0; j < C::WN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][e], b[j][e], acc[i][j], 0, 0, 0);
  }
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

// Software pipeline over ntiles k-tiles: tile t+1 and t+2 are in flight in
// two register sets while tile t is multiplied from LDS (double-buffered, one
// barrier per k-tile).  The stage supplies load<S>(t) (global -> register set
// S) and store<S>(buf) (register set S -> an LDS buffer of LDS_FLOATS, A tile
// then B tile); the loop is unrolled by two so the sets alternate statically.
// The loop body runs whole tile pairs and has no exit in its middle, and an
// odd last tile is done after it: with a single exit the accumulators keep
// one register assignment around the loop (a mid-body exit made the compiler
// copy every accumulator between two register sets each iteration).
// Ends with a barrier, after which lds may be reused.
template <class C, class Stage>
__device__ __forceinline__ void pipeline(int ntiles, float* lds, Stage& s,
                                         f32x16 (&acc)[C::WM][C::WN]) {
  float* buf0 = lds;
  float* buf1 = lds + C::LDS_FLOATS;
  constexpr int BOFF = C::BM * C::LDK;
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
    mfma_ktile<C>(buf0, buf0 + BOFF, acc);
    s.template store<0>(buf1);
    if (kt + 3 < ntiles) s.template load<0>(kt + 3);
    __syncthreads();
    // tile kt+1 in buf1, kt+2 in set 1, kt+3 in set 0
    mfma_ktile<C>(buf1, buf1 + BOFF, acc);
    if (kt + 2 < ntiles) {
      s.template store<1>(buf0);
      if (kt + 4 < ntiles) s.template load<1>(kt + 4);
    }
    __syncthreads();
  }
  if (kt < ntiles) {  // odd count: the last tile is in buf0
    mfma_ktile<C>(buf0, buf0 + BOFF, acc);
    __syncthreads();
  }
}

}  // namespace kp
}  // namespace cnhip
