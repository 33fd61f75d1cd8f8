// fp32 GEMM on CDNA4 matrix cores (v_mfma_f32_32x32x2f32), ColMajor operands.
//
//   C[M,N] = alpha * op(A)[M,K] * op(B)[K,N] + beta * C (+ bias[n]) (ReLU)
//
// One kernel template covers the three shapes a Linear layer needs
// (forward NN, weight-grad TN, input-grad NT; ref: matmul.cu:16-71,
// matmul_grad_weight.cu:14-69, matmul_grad_input.cu:14-68) and the batched
// products of the recurrent and attention layers.  The reference computes one
// output per thread with atomicAdd accumulation.  Here a block of
// WGM x WGN wave64s owns a (WGM*WM*32) x (WGN*WN*32) output tile (up to
// 256 x 128, each wave 128 x 64 as 4 x 2 MFMA blocks); K advances 16 at a
// time through double-buffered, k-contiguous LDS tiles (mfma_kpack.hpp); no
// atomics are used.  When the output tiles alone cannot fill the 256 CUs, K
// is split across blocks into a stream-ordered workspace and the partials
// are summed in a fixed order, so results are deterministic.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <vector>

#include "act_math.hpp"
#include "colsum.hpp"
#include "common.hpp"
#include "mfma_kpack.hpp"

namespace cnhip {
namespace {

using kp::f32x16;
using kp::f32x4;

// Tile shapes (measured on MI355X: the 8-wave blocks keep two waves per SIMD
// with 64x64 wave tiles and beat 4-wave blocks with larger wave tiles).
using CfgXL = kp::Cfg<4, 2, 2, 2>;  // 256 x 128, 8 waves of 64x64
using CfgXN = kp::Cfg<2, 4, 2, 2>;  // 128 x 256, 8 waves of 64x64
using CfgXX = kp::Cfg<4, 4, 2, 2>;  // 256 x 256, 16 waves of 64x64 (one block per CU)
using CfgM = kp::Cfg<4, 2, 1, 2>;   // 128 x 128, 8 waves of 32x64
using CfgSN = kp::Cfg<4, 1, 1, 1>;  // 128 x 32 : N <= 32
using CfgSM = kp::Cfg<1, 4, 1, 1>;  // 32 x 128 : M <= 32
using CfgS = kp::Cfg<2, 2, 1, 1>;   // 64 x 64  : small problems

// Split-K granularity: a multiple of every tile shape's BK.
constexpr int64_t KQ = 32;

// Blocks of 512 threads run one per CU (their 64x64 wave tiles need ~150
// VGPRs); 256-thread blocks are sized for two.
template <class C>
constexpr int min_blocks() { return C::NT >= 512 ? 4 : 2; }

struct GemmArgs {
  int64_t M, N, K;
  const float* A;
  int64_t lda, stride_a;  // stride_a: elements between batch entries
  const float* B;
  int64_t ldb, stride_b;
  float* C;
  int64_t ldc, stride_c;
  float alpha, beta;
  const float* bias;
  int epilogue;          // CNHIP_EPI_* or one of the fused-activation codes below
  const float* aux_in;   // DRELU: ReLU outputs, DGELU: GELU inputs, [M,N] ld ld_aux
  float* aux_out;        // GELU: receives the pre-activation, [M,N] ld ld_aux
  int64_t ld_aux;
  int vec_ok;            // every ld and stride % 4 == 0 and A, B 16-byte aligned
  int c_vec_ok;          // ldc, stride_c % 4 == 0 and C 16-byte aligned
  int aux_vec_ok;        // ld_aux % 4 == 0 and aux_in 16-byte aligned
  int64_t k_per_split;   // multiple of KQ (hence of every tile's BK)
  float* partial;        // split-K workspace [batch][splits][M*N]; null = direct
  int splits;
  float* colsum;         // small kernels only: colsum[n] (+)= sum_k op(B)(k, n), or null
  int colsum_acc;        // 1: add to colsum, 0: overwrite
};

// Fused-activation epilogues (internal codes beyond the C ABI's NONE / RELU):
//   EPI_GELU : C = gelu(v), aux_out = v (the pre-activation GELU's backward reads)
//   EPI_DRELU: C = v * [aux_in > 0]      (ReLU backward on the layer below)
//   EPI_DGELU: C = v * gelu'(aux_in)     (GELU backward on the layer below)
//   EPI_ADD  : C = v + aux_in            (a residual branch added to the output)
//   EPI_TANH : C = tanh(v)               (the Elman RNN cell)
// where v = alpha * acc (+ beta * C) (+ bias[n]).
constexpr int EPI_GELU = 2, EPI_DRELU = 3, EPI_DGELU = 4, EPI_ADD = 5, EPI_TANH = 6;

// FUSED: the kernel instantiation that also handles the fused-activation
// codes; the plain one (the bulk of all launches) keeps its epilogue small so
// its code stays compact.
template <bool FUSED>
__device__ __forceinline__ float epilogue_value(const GemmArgs& g, const float* C, float acc,
                                                int64_t m, int64_t n) {
  float v = g.alpha * acc;
  if (g.beta != 0.f) v += g.beta * C[m + g.ldc * n];
  if (g.bias) v += g.bias[n];
  if (!FUSED) return g.epilogue == CNHIP_EPI_RELU ? relu_f(v) : v;
  switch (g.epilogue) {
    case CNHIP_EPI_RELU: return relu_f(v);
    case EPI_GELU:
      g.aux_out[m + g.ld_aux * n] = v;
      return gelu_f(v);
    case EPI_DRELU: return v * relu_mask(g.aux_in[m + g.ld_aux * n]);
    case EPI_DGELU: return v * gelu_grad_f(g.aux_in[m + g.ld_aux * n]);
    case EPI_ADD: return v + g.aux_in[m + g.ld_aux * n];
    case EPI_TANH: return tanhf(v);
    default: return v;
  }
}

// Block -> output tile.  Hardware dispatch places consecutive block ids on
// consecutive XCDs (8 of them, each with its own L2); remap so that every XCD
// owns a contiguous range of tiles, then walk tiles in groups of 8 tile-rows
// so neighbouring blocks on one XCD share A rows and B columns in its L2.
__device__ __forceinline__ void tile_of_block(int bid, int nbm, int nbn, int& tm, int& tn) {
  const int total = nbm * nbn;
  const int xcd = bid & 7, local = bid >> 3;
  const int base = total >> 3, rem = total & 7;
  const int tile = xcd * base + min(xcd, rem) + local;
  constexpr int GROUP = 8;
  const int per_group = GROUP * nbn;
  const int group = tile / per_group;
  const int first_m = group * GROUP;
  const int gsz = min(nbm - first_m, GROUP);
  const int in_group = tile - group * per_group;
  tm = first_m + in_group % gsz;
  tn = in_group / gsz;
}

// Global -> LDS staging of one GEMM block for kp::pipeline (global loads two
// k-tiles ahead of the MFMAs through two register sets, double-buffered LDS,
// one barrier per k-tile).
template <bool FAST, bool TA, bool TB, class C>
struct GemmStage {
  using OA = kp::Operand<TA, C::BM, C::NT, C::BK>;   // A(m,k): k-contiguous when A is transposed
  using OB = kp::Operand<!TB, C::BN, C::NT, C::BK>;  // B(k,n): k-contiguous unless B is transposed
  const GemmArgs& g;
  const float* A;
  const float* B;
  int64_t m0, n0, k_begin, k_end;
  f32x4 ra[2][OA::REGS], rb[2][OB::REGS];

  __device__ GemmStage(const GemmArgs& g_, const float* A_, const float* B_, int64_t m0_,
                       int64_t n0_, int64_t kb, int64_t ke)
      : g(g_), A(A_), B(B_), m0(m0_), n0(n0_), k_begin(kb), k_end(ke) {}

  template <int S>
  __device__ __forceinline__ void load(int t) {
    const int64_t k0 = k_begin + (int64_t)t * C::BK;
    OA::template load<FAST>(A, g.lda, m0, k0, g.M, k_end, ra[S]);
    OB::template load<FAST>(B, g.ldb, n0, k0, g.N, k_end, rb[S]);
  }
  template <int S>
  __device__ __forceinline__ void store(float* buf) {
    OA::store(buf, ra[S]);
    OB::store(buf + OA::FLOATS, rb[S]);
  }
};

// K loop of one block over [k_begin, k_end) on the shared MFMA pipeline.
// FAST: every tile load is in range and 16-byte aligned (no per-element
// checks).
template <bool FAST, bool TA, bool TB, class C>
__device__ __forceinline__ void gemm_mainloop(const GemmArgs& g, const float* __restrict__ A,
                                              const float* __restrict__ B, int64_t m0, int64_t n0,
                                              int64_t k_begin, int64_t k_end, float* lds,
                                              f32x16 (&acc)[C::WM][C::WN]) {
  const int ntiles = k_end > k_begin ? (int)((k_end - k_begin + C::BK - 1) / C::BK) : 0;
  GemmStage<FAST, TA, TB, C> s(g, A, B, m0, n0, k_begin, k_end);
  kp::pipeline<C>(ntiles, lds, s, acc);
}

// Epilogue of an interior tile (every row and column in range, C float4-
// aligned, beta == 0, no split-K).  AUX: the fused epilogue reads aux_in
// (DRELU, DGELU, ADD; aux_in float4-aligned), else it is NONE or RELU.
// The pointers are __restrict__ so loads may be scheduled ahead of stores
// to C: the bias of every column the thread owns is loaded first, and per
// 32 x 32 accumulator block the four aux float4s are loaded before the
// block's results are stored, the next block's before this block's stores.
// (Through possibly aliasing pointers every load waited for the previous
// store, and the epilogue paid the memory latency once per float4.)  The
// arithmetic per element is epilogue_value's.
template <class C, bool AUX>
__device__ __forceinline__ void epilogue_interior(const GemmArgs& g, float* __restrict__ Cp,
                                                  const float* __restrict__ aux,
                                                  const float* __restrict__ bias,
                                                  const f32x16 (&acc)[C::WM][C::WN], int64_t m0,
                                                  int64_t n0) {
  const int lane = threadIdx.x & 63;
  int wm, wn, wk;
  kp::wave_pos<C>(wm, wn, wk);
  if (C::WGK > 1 && wk != 0) return;
  constexpr int NB = C::WM * C::WN;
  auto col = [&](int b) { return n0 + wn * (C::WN * 32) + (b % C::WN) * 32 + (lane & 31); };
  auto row = [&](int b, int q) { return m0 + wm * (C::WM * 32) + (b / C::WN) * 32 + 8 * q + 4 * (lane >> 5); };
  float bv[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) bv[b] = bias ? bias[col(b)] : 0.f;
  f32x4 cur[4], nxt[4];
  if constexpr (AUX) {
#pragma unroll
    for (int q = 0; q < 4; ++q) cur[q] = *reinterpret_cast<const f32x4*>(aux + row(0, q) + g.ld_aux * col(0));
  }
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    if constexpr (AUX) {
      if (b + 1 < NB) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          nxt[q] = *reinterpret_cast<const f32x4*>(aux + row(b + 1, q) + g.ld_aux * col(b + 1));
      }
    }
    const int64_t n = col(b);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      f32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float v = g.alpha * acc[b / C::WN][b % C::WN][4 * q + e];
        if (bias) v += bv[b];
        if constexpr (AUX) {
          const float a = cur[q][e];
          o[e] = g.epilogue == EPI_DRELU   ? v * relu_mask(a)
                 : g.epilogue == EPI_DGELU ? v * gelu_grad_f(a)
                                           : v + a;
        } else {
          o[e] = g.epilogue == CNHIP_EPI_RELU ? relu_f(v) : v;
        }
      }
      *reinterpret_cast<f32x4*>(Cp + row(b, q) + g.ldc * n) = o;
    }
    if constexpr (AUX) {
      if (b + 1 < NB) {
#pragma unroll
        for (int q = 0; q < 4; ++q) cur[q] = nxt[q];
      }
    }
  }
}

template <bool TA, bool TB, class C>
constexpr int gemm_lds_floats() {
  return 2 * kp::stage_floats<GemmStage<true, TA, TB, C>>();
}

// One block of a GEMM launch: tile block `bx` (grid x), batch entry `batch`
// (grid y) and k-split `split` (grid z).
template <bool TA, bool TB, class C, bool FUSED>
__device__ __forceinline__ void gemm_block(const GemmArgs& g, float* lds, int bx, int64_t batch, int split) {
  constexpr int BM = C::BM, BN = C::BN;
  const int nbm = (int)((g.M + BM - 1) / BM);
  const int nbn = (int)((g.N + BN - 1) / BN);
  int tm, tn;
  tile_of_block(bx, nbm, nbn, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const float* A = g.A + batch * g.stride_a;
  const float* B = g.B + batch * g.stride_b;

  const int64_t k_begin = (int64_t)split * g.k_per_split;
  const int64_t k_end = min(g.K, k_begin + g.k_per_split);
  const bool full_mn = (m0 + BM <= g.M) && (n0 + BN <= g.N);
  const bool fast = g.vec_ok && full_mn && ((k_end - k_begin) % C::BK == 0);

  f32x16 acc[C::WM][C::WN];
  kp::zero_acc<C>(acc);
  if (fast) gemm_mainloop<true, TA, TB, C>(g, A, B, m0, n0, k_begin, k_end, lds, acc);
  else gemm_mainloop<false, TA, TB, C>(g, A, B, m0, n0, k_begin, k_end, lds, acc);

  float* Cp = g.C + batch * g.stride_c;
  if (full_mn && g.c_vec_ok && !g.partial && g.beta == 0.f) {
    if constexpr (FUSED) {
      if ((g.epilogue == EPI_DRELU || g.epilogue == EPI_DGELU || g.epilogue == EPI_ADD) && g.aux_vec_ok) {
        epilogue_interior<C, true>(g, Cp, g.aux_in, g.bias, acc, m0, n0);
        return;
      }
    } else {
      epilogue_interior<C, false>(g, Cp, nullptr, g.bias, acc, m0, n0);
      return;
    }
  }
  float* P = g.partial ? g.partial + (batch * g.splits + split) * g.M * g.N : nullptr;
  const bool p_vec = (g.M & 3) == 0;
  kp::for_each_acc_run<C>(acc, [&](int ml, int nl, const f32x4& v) {
    const int64_t m = m0 + ml, n = n0 + nl;
    if (n >= g.N) return;
    if (P) {
      if (p_vec && m + 3 < g.M) {
        *reinterpret_cast<f32x4*>(P + m + g.M * n) = v;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (m + e < g.M) P[(m + e) + g.M * n] = v[e];
      }
      return;
    }
    if (g.c_vec_ok && m + 3 < g.M) {
      f32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = epilogue_value<FUSED>(g, Cp, v[e], m + e, n);
      *reinterpret_cast<f32x4*>(Cp + m + g.ldc * n) = o;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (m + e < g.M) Cp[(m + e) + g.ldc * n] = epilogue_value<FUSED>(g, Cp, v[e], m + e, n);
    }
  });
}

template <bool TA, bool TB, class C, bool FUSED>
__global__ void __launch_bounds__(C::NT, min_blocks<C>()) gemm_f32_kernel(GemmArgs g) {
  __shared__ __align__(16) float lds[gemm_lds_floats<TA, TB, C>()];
  gemm_block<TA, TB, C, FUSED>(g, lds, (int)blockIdx.x, (int64_t)blockIdx.y, (int)blockIdx.z);
}

// Two independent GEMMs in one launch, both on tile shape C: blocks
// [0, n1) run the first's (tiles1 x batches1 x splits1) blocks, the rest the
// second's, each block exactly as in its own launch (so each product is
// bit-identical to a launch of its own with the same plan).  A GEMM whose
// tiles fill only one of the two block slots per CU (256 tiles of 128 x 128)
// leaves every CU's matrix pipe idle while its single block loads its first
// k-tiles and stores its results; a second GEMM's blocks in the other slot
// fill those gaps.
template <bool TA1, bool TB1, bool F1, bool TA2, bool TB2, bool F2, class C>
__global__ void __launch_bounds__(C::NT, min_blocks<C>()) gemm_pair_kernel(GemmArgs g1, GemmArgs g2, int n1,
                                                                           int tiles1, int batches1, int tiles2,
                                                                           int batches2) {
  constexpr int F = gemm_lds_floats<TA1, TB1, C>() > gemm_lds_floats<TA2, TB2, C>()
                        ? gemm_lds_floats<TA1, TB1, C>()
                        : gemm_lds_floats<TA2, TB2, C>();
  __shared__ __align__(16) float lds[F];
  int b = (int)blockIdx.x;
  if (b < n1) {
    gemm_block<TA1, TB1, C, F1>(g1, lds, b % tiles1, (b / tiles1) % batches1, b / (tiles1 * batches1));
  } else {
    b -= n1;
    gemm_block<TA2, TB2, C, F2>(g2, lds, b % tiles2, (b / tiles2) % batches2, b / (tiles2 * batches2));
  }
}

// Sums split-K partials in split order and applies the epilogue.
__global__ void __launch_bounds__(256) splitk_reduce_kernel(GemmArgs g, int64_t batches) {
  const int64_t mn = g.M * g.N;
  const int64_t total = mn * batches;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t bt = idx / mn, e = idx - bt * mn;
    const float* P = g.partial + bt * g.splits * mn + e;
    // unrolled so the loads issue ahead; the additions stay in split order
    float s = 0.f;
#pragma unroll 8
    for (int z = 0; z < g.splits; ++z) s += P[(int64_t)z * mn];
    const int64_t m = e % g.M, n = e / g.M;
    float* C = g.C + bt * g.stride_c;
    C[m + g.ldc * n] = epilogue_value<true>(g, C, s, m, n);
  }
}

// Tiny GEMMs (a few MFLOP: the 30-64-1 MLP's layers, a classifier head) are
// latency-bound: an MFMA tile's k-loop and a split-K reduce launch cost more
// than the arithmetic.  These SIMT kernels compute each output with plain
// fp32 FMAs and the same epilogue as the tiled kernel (batches == 1).
//   gemm_small_thread_kernel: one thread per output, k from 0 to K-1 (K <= 64);
//   gemm_small_wave_kernel:   one wave per output, lane l takes k = l, l+64, ...
//                             in order, then a fixed butterfly over the lanes.
template <bool TA, bool TB>
__device__ __forceinline__ float op_a(const GemmArgs& g, int64_t m, int64_t k) {
  return TA ? g.A[k + g.lda * m] : g.A[m + g.lda * k];
}
template <bool TA, bool TB>
__device__ __forceinline__ float op_b(const GemmArgs& g, int64_t k, int64_t n) {
  return TB ? g.B[n + g.ldb * k] : g.B[k + g.ldb * n];
}

// With g.colsum set (a Linear layer's weight gradient, op(B) = dY), the
// outputs of row m = 0 also sum their op(B) column: the bias gradient in the
// same launch.
template <bool TA, bool TB>
__device__ __forceinline__ void small_thread_block(const GemmArgs& g, int64_t bid) {
  const int64_t e = bid * 256 + threadIdx.x;
  if (e >= g.M * g.N) return;
  const int64_t m = e % g.M, n = e / g.M;
  const bool cs = g.colsum && m == 0;
  float acc = 0.f, sum = 0.f;
  // unrolled so the loads issue ahead; the FMAs stay in k order
#pragma unroll 8
  for (int64_t k = 0; k < g.K; ++k) {
    const float b = op_b<TA, TB>(g, k, n);
    acc = fmaf(op_a<TA, TB>(g, m, k), b, acc);
    if (cs) sum += b;
  }
  g.C[m + g.ldc * n] = epilogue_value<true>(g, g.C, acc, m, n);
  if (cs) g.colsum[n] = g.colsum_acc ? g.colsum[n] + sum : sum;
}

template <bool TA, bool TB>
__global__ void __launch_bounds__(256) gemm_small_thread_kernel(GemmArgs g) {
  small_thread_block<TA, TB>(g, blockIdx.x);
}

template <bool TA, bool TB>
__device__ __forceinline__ void small_wave_block(const GemmArgs& g, int64_t bid) {
  const int64_t e = bid * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (e >= g.M * g.N) return;  // uniform per wave
  const int64_t m = e % g.M, n = e / g.M;
  const bool cs = g.colsum && m == 0;  // uniform per wave
  float acc = 0.f, sum = 0.f;
#pragma unroll 4
  for (int64_t k = lane; k < g.K; k += 64) {
    const float b = op_b<TA, TB>(g, k, n);
    acc = fmaf(op_a<TA, TB>(g, m, k), b, acc);
    if (cs) sum += b;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (cs) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
  }
  if (lane == 0) {
    g.C[m + g.ldc * n] = epilogue_value<true>(g, g.C, acc, m, n);
    if (cs) g.colsum[n] = g.colsum_acc ? g.colsum[n] + sum : sum;
  }
}

template <bool TA, bool TB>
__global__ void __launch_bounds__(256) gemm_small_wave_kernel(GemmArgs g) {
  small_wave_block<TA, TB>(g, blockIdx.x);
}

// A small Linear layer's weight gradient (with its bias sums) and input
// gradient in one launch: blocks [0, n1) are the first's, the rest the
// second's, each block computing exactly as in its own launch.
template <bool W1, bool W2>
__global__ void __launch_bounds__(256) gemm_small_pair_kernel(GemmArgs g1, GemmArgs g2, int64_t n1) {
  const int64_t b = blockIdx.x;
  if (b < n1) {
    if (W1) small_wave_block<true, false>(g1, b);
    else small_thread_block<true, false>(g1, b);
  } else {
    if (W2) small_wave_block<false, true>(g2, b - n1);
    else small_thread_block<false, true>(g2, b - n1);
  }
}

// splitk_reduce_kernel for M % 4 == 0 and fewer than 2^31 outputs: float4
// partial loads (four consecutive m share n), 32-bit index arithmetic; the
// same split-order sums and epilogue per element.
__device__ __forceinline__ void splitk_reduce_vec(const GemmArgs& g, int batches, uint32_t first, uint32_t stride) {
  const uint32_t M = (uint32_t)g.M, mn4 = (uint32_t)(g.M * g.N) >> 2;
  const uint32_t total4 = mn4 * (uint32_t)batches;
  const int64_t mn = g.M * g.N;
  for (uint32_t q = first; q < total4; q += stride) {
    const uint32_t bt = batches == 1 ? 0u : q / mn4;
    const uint32_t e = (q - bt * mn4) << 2;
    const f32x4* P = reinterpret_cast<const f32x4*>(g.partial + (int64_t)bt * g.splits * mn + e);
    const int64_t zs = mn >> 2;
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
    for (int z = 0; z < g.splits; ++z) s += P[z * zs];
    const uint32_t n = e / M, m = e - n * M;
    float* C = g.C + (int64_t)bt * g.stride_c;
    f32x4 o;
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = epilogue_value<true>(g, C, s[k], m + k, n);
    if (g.c_vec_ok) {
      *reinterpret_cast<f32x4*>(C + m + g.ldc * n) = o;
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) C[(m + k) + g.ldc * n] = o[k];
    }
  }
}

__global__ void __launch_bounds__(256) splitk_reduce_vec_kernel(GemmArgs g, int batches) {
  splitk_reduce_vec(g, batches, blockIdx.x * blockDim.x + threadIdx.x, gridDim.x * blockDim.x);
}

// The split-K reduce above in blocks [0, rblocks) and, in the rest, the
// column sums of an independent matrix (a Linear's bias gradient), one wave
// per column as column_sum does: two bandwidth-bound passes of a few
// microseconds each in one launch.
__global__ void __launch_bounds__(256) splitk_reduce_colsum_kernel(GemmArgs g, int batches, int rblocks, ColsumJob cs) {
  if ((int)blockIdx.x < rblocks) {
    splitk_reduce_vec(g, batches, blockIdx.x * blockDim.x + threadIdx.x, (uint32_t)rblocks * blockDim.x);
    return;
  }
  colsum_wave(cs, (int64_t)(blockIdx.x - rblocks) * 4 + (threadIdx.x >> 6), threadIdx.x & 63);
}

template <bool TA, bool TB, class Cfg>
void launch_cfg(const GemmArgs& g, int64_t batches, hipStream_t st) {
  const int64_t tiles = ((g.M + Cfg::BM - 1) / Cfg::BM) * ((g.N + Cfg::BN - 1) / Cfg::BN);
  const dim3 grid((unsigned)tiles, (unsigned)batches, (unsigned)g.splits);
  // the fused-activation epilogues are only used by the forward (NN) and
  // input-gradient (NT) GEMMs of Linear layers
  constexpr bool kFusable = !TA;
  if (kFusable && g.epilogue >= EPI_GELU && !g.partial)
    hipLaunchKernelGGL((gemm_f32_kernel<TA, TB, Cfg, kFusable>), grid, dim3(Cfg::NT), 0, st, g);
  else
    hipLaunchKernelGGL((gemm_f32_kernel<TA, TB, Cfg, false>), grid, dim3(Cfg::NT), 0, st, g);
}

template <class Cfg>
void launch_t(int ta, int tb, const GemmArgs& g, int64_t batches, hipStream_t st) {
  if (!ta && !tb) launch_cfg<false, false, Cfg>(g, batches, st);
  else if (ta && !tb) launch_cfg<true, false, Cfg>(g, batches, st);
  else if (!ta && tb) launch_cfg<false, true, Cfg>(g, batches, st);
  else launch_cfg<true, true, Cfg>(g, batches, st);
}

// Per-launch event timing (cnhip_gemm_timing_*): a pool of event pairs
// reused across enable() calls.
struct Timing {
  bool on = false;
  std::vector<TimingRec> pool;
  size_t used = 0;
};
thread_local Timing g_timing;      // MFMA GEMM-shaped launches
thread_local Timing g_hbm_timing;  // bandwidth-bound launches

TimingRec* next_slot(Timing& t) {
  if (!t.on || fixed_scratch_active()) return nullptr;
  if (t.used == t.pool.size()) {
    TimingRec r{};
    // timing-only events: no system-scope fence (cache writeback) at record,
    // which would add to the duration of short launches
    if (hipEventCreateWithFlags(&r.start, hipEventDisableSystemFence) != hipSuccess ||
        hipEventCreateWithFlags(&r.stop, hipEventDisableSystemFence) != hipSuccess) {
      (void)hipGetLastError();
      return nullptr;
    }
    t.pool.push_back(r);
  }
  return &t.pool[t.used++];
}

}  // namespace

bool timing_on() { return g_timing.on || g_hbm_timing.on; }

TimingRec* timing_slot(double flops) {
  TimingRec* r = next_slot(g_timing);
  if (r) {
    r->flops = flops;
    r->kernel = nullptr;
    r->bytes = 0.0;
  }
  return r;
}

TimingRec* hbm_timing_slot(const char* kernel, double bytes) {
  TimingRec* r = next_slot(g_hbm_timing);
  if (r) {
    r->flops = 0.0;
    r->kernel = kernel;
    r->bytes = bytes;
  }
  return r;
}

namespace {

enum class Shape { XX, XL, XN, M, SN, SM, S };

template <class Cfg>
int64_t tiles_of(int64_t M, int64_t N) {
  return ((M + Cfg::BM - 1) / Cfg::BM) * ((N + Cfg::BN - 1) / Cfg::BN);
}

struct Plan {
  Shape shape;
  int64_t tiles;
  int splits;
  int64_t kps;
};

// Tile shape and split-K plan of one GEMM; splits <= max_splits.
// Cost model of one launch: dispatch rounds times the K-tiles of one split,
// plus the fixed-order reduce of split-K partials (read splits + 1 times M*N
// floats at ~5 TB/s, and a launch).  Block slots per round: the 512-thread
// shapes are compiled for 4 waves per SIMD, so 2 blocks share a CU (512
// slots); the 256-thread 64 x 64 and skinny tiles fit 4 per CU (1024).  A
// split count that leaves a nearly empty last round costs a whole extra
// round, so it is avoided.  `eff` is the measured MFMA efficiency of the
// tile relative to the 64 x 64-per-wave tiles (smaller per-wave tiles load
// more LDS bytes per MFMA).  Splits keep >= 4 K-tiles of 32.  Returns the
// estimated seconds and the best split count.
double split_cost(Shape shape, int64_t tiles, int64_t M, int64_t N, int64_t K, int64_t batches,
                  int max_splits, bool may_split, int& splits) {
  int64_t bm = 0, bn = 0;
  double eff = 1.0;
  switch (shape) {
    case Shape::XX: bm = CfgXX::BM; bn = CfgXX::BN; break;
    case Shape::XL: bm = CfgXL::BM; bn = CfgXL::BN; break;
    case Shape::XN: bm = CfgXN::BM; bn = CfgXN::BN; break;
    case Shape::M: bm = CfgM::BM; bn = CfgM::BN; eff = 0.95; break;
    case Shape::SN: bm = CfgSN::BM; bn = CfgSN::BN; eff = 0.8; break;
    case Shape::SM: bm = CfgSM::BM; bn = CfgSM::BN; eff = 0.8; break;
    case Shape::S: bm = CfgS::BM; bn = CfgS::BN; eff = 0.8; break;
  }
  const bool big = shape == Shape::XX || shape == Shape::XL || shape == Shape::XN || shape == Shape::M;
  const int64_t per_cu = big ? 2 : 4;
  const int64_t slots = 256 * per_cu;
  // seconds per K-tile of 32 of one block, sharing its CU with per_cu - 1 others
  const double t_tile = 2.0 * bm * bn * KQ / (157.3e12 / 256) * (double)per_cu / eff;
  const int64_t blocks = tiles * batches;
  int64_t max_s = 1;
  if (may_split && blocks < slots && K >= 8 * KQ)
    max_s = std::max<int64_t>(1, std::min<int64_t>(K / (4 * KQ), max_splits));
  double best = 0.0;
  splits = 1;
  for (int64_t s = 1; s <= max_s; ++s) {
    const int64_t kt = ((K + s - 1) / s + KQ - 1) / KQ;
    const int64_t rounds = (blocks * s + slots - 1) / slots;
    double cost = (double)rounds * (double)kt * t_tile;
    if (s > 1) cost += (double)(s + 1) * M * N * batches * 4.0 / 5e12 + 3e-6;
    if (s == 1 || cost < best) {
      best = cost;
      splits = (int)s;
    }
  }
  return best;
}

Plan plan_gemm(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, int64_t batches,
               int max_splits) {
  // Skinny shapes take the 32-wide tiles (no MFMA work on padding), split by
  // the cost model above.  Otherwise, in order (rules fitted to measured
  // tile x split sweeps on MI355X, where the 512-thread tiles run 2 blocks
  // per CU and split-K costs more than its reduce traffic alone):
  //   128 x 256 (256 x 128 when only A is k-contiguous) if >= 512 blocks,
  //   256 x 256 instead when that gives whole rounds of 256 blocks, K >= 1024;
  //   128 x 128 if >= 256 blocks;  64 x 64 if >= 512 blocks;
  //   else split K: 128 x 128 toward 512 blocks (<= 16 splits) if that
  //   reaches 256 blocks, otherwise 64 x 64 toward 512 blocks.
  Shape shape;
  int splits = 1;
  if (N <= 32 || M <= 32) {
    shape = N <= 32 ? Shape::SN : Shape::SM;
    split_cost(shape, shape == Shape::SN ? tiles_of<CfgSN>(M, N) : tiles_of<CfgSM>(M, N), M, N, K,
               batches, max_splits, true, splits);
  } else {
    const bool a_kc = trans_a != 0, b_kc = trans_b == 0;
    const Shape big = (a_kc && !b_kc) ? Shape::XL : Shape::XN;
    const int64_t tb = (big == Shape::XL ? tiles_of<CfgXL>(M, N) : tiles_of<CfgXN>(M, N)) * batches;
    const int64_t tm = tiles_of<CfgM>(M, N) * batches;
    const int64_t ts = tiles_of<CfgS>(M, N) * batches;
    const int64_t max_s = K >= 8 * KQ ? std::max<int64_t>(1, std::min<int64_t>(K / (4 * KQ), max_splits)) : 1;
    if (tb >= 512) {
      // whole rounds of 256 x 256 tiles (one 16-wave block per CU) for a
      // long contraction: each staged k-tile feeds 16 waves instead of 8
      // (config 2's 4096^3 GEMMs 0.6-1.7% faster than 128 x 256)
      const int64_t tx = tiles_of<CfgXX>(M, N) * batches;
      shape = K >= 1024 && tx % 256 == 0 ? Shape::XX : big;
    } else if (tm >= 256) {
      shape = Shape::M;
    } else if (ts >= 512) {
      shape = Shape::S;
    } else {
      // too few tiles to fill the chip: split K.  The 128 x 128 tile's split
      // count (<= 16) is the one with the lowest dispatch-round cost: a count
      // that leaves some CUs a block more than the others costs that block's
      // whole duration (11 splits of 48 tiles, 528 blocks, ran at 82 TFLOP/s
      // where 10 splits, 480 blocks, run at 92)
      int sm = 1;
      split_cost(Shape::M, tm / batches, M, N, K, batches, (int)std::min<int64_t>(16, max_s), true, sm);
      if (tm * sm >= 256) {
        shape = Shape::M;
        splits = sm;
      } else {
        shape = Shape::S;
        splits = (int)std::min<int64_t>((512 + ts - 1) / ts, max_s);
      }
    }
  }
  int64_t tiles = 0;
  switch (shape) {
    case Shape::XX: tiles = tiles_of<CfgXX>(M, N); break;
    case Shape::XL: tiles = tiles_of<CfgXL>(M, N); break;
    case Shape::XN: tiles = tiles_of<CfgXN>(M, N); break;
    case Shape::M: tiles = tiles_of<CfgM>(M, N); break;
    case Shape::SN: tiles = tiles_of<CfgSN>(M, N); break;
    case Shape::SM: tiles = tiles_of<CfgSM>(M, N); break;
    case Shape::S: tiles = tiles_of<CfgS>(M, N); break;
  }
  int64_t kps = (K + splits - 1) / splits;
  kps = ((kps + KQ - 1) / KQ) * KQ;
  if (kps == 0) kps = KQ;
  splits = K > 0 ? (int)((K + kps - 1) / kps) : 1;

  return Plan{shape, tiles, splits, kps};
}

// Launches the planned kernel, bracketed by the per-launch timing events.
int launch_plan(Shape shape, int trans_a, int trans_b, const GemmArgs& g, int64_t batches,
                hipStream_t st, const char* who) {
  TimingRec* rec =
      timing_slot(2.0 * (double)g.M * (double)g.N * (double)g.K * (double)batches);
  if (rec) (void)hipEventRecord(rec->start, st);
  switch (shape) {
    case Shape::XX: launch_t<CfgXX>(trans_a, trans_b, g, batches, st); break;
    case Shape::XL: launch_t<CfgXL>(trans_a, trans_b, g, batches, st); break;
    case Shape::XN: launch_t<CfgXN>(trans_a, trans_b, g, batches, st); break;
    case Shape::M: launch_t<CfgM>(trans_a, trans_b, g, batches, st); break;
    case Shape::SN: launch_t<CfgSN>(trans_a, trans_b, g, batches, st); break;
    case Shape::SM: launch_t<CfgSM>(trans_a, trans_b, g, batches, st); break;
    case Shape::S: launch_t<CfgS>(trans_a, trans_b, g, batches, st); break;
  }
  const int status = check_launch(who);
  if (rec) (void)hipEventRecord(rec->stop, st);
  return status;
}

}  // namespace

// Single GEMM with a fused-activation epilogue (see epilogue_value):
// aux is [M,N] with leading dimension ld_aux (an output for EPI_GELU, an
// input for EPI_DRELU / EPI_DGELU / EPI_ADD).
int gemm_f32_act(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, const float* A,
                 int64_t lda, const float* B, int64_t ldb, float* C, int64_t ldc, const float* bias,
                 int epilogue, const float* aux_in, float* aux_out, int64_t ld_aux, hipStream_t st,
                 const char* who);

int gemm_f32_core(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha,
                  const float* A, int64_t lda, int64_t stride_a, const float* B, int64_t ldb,
                  int64_t stride_b, float beta, float* C, int64_t ldc, int64_t stride_c,
                  int64_t batches, const float* bias, int epilogue, const float* aux_in,
                  float* aux_out, int64_t ld_aux, hipStream_t st, const char* who);

int gemm_f32_batched(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha,
                     const float* A, int64_t lda, int64_t stride_a, const float* B, int64_t ldb,
                     int64_t stride_b, float beta, float* C, int64_t ldc, int64_t stride_c,
                     int64_t batches, const float* bias, int epilogue, hipStream_t st,
                     const char* who) {
  CNHIP_REQUIRE(epilogue == CNHIP_EPI_NONE || epilogue == CNHIP_EPI_RELU, "%s: bad epilogue %d",
                who, epilogue);
  return gemm_f32_core(trans_a, trans_b, M, N, K, alpha, A, lda, stride_a, B, ldb, stride_b, beta,
                       C, ldc, stride_c, batches, bias, epilogue, nullptr, nullptr, 0, st, who);
}

// GEMMs up to this many flops and outputs take the SIMT kernels above
constexpr double kSmallGemmFlops = 4.0e6;
constexpr int64_t kSmallGemmOutputs = 1 << 16;

// Weight-gradient shapes (op(A) = A^T, A k-contiguous; B not transposed, also
// k-contiguous) read whole contiguous k-runs per wave, so the wave kernel
// stays efficient up to this many flops (a skinny classifier's dW).
constexpr double kSmallWgradFlops = 32.0e6;

static bool gemm_is_small(int64_t M, int64_t N, int64_t K, int64_t batches, int trans_a = 0,
                          int trans_b = 0) {
  if (batches != 1 || K <= 0 || M * N > kSmallGemmOutputs) return false;
  const double flops = 2.0 * (double)M * (double)N * (double)K;
  return flops <= kSmallGemmFlops || (trans_a && !trans_b && K > 64 && flops <= kSmallWgradFlops);
}

static int gemm_small(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha,
                      const float* A, int64_t lda, const float* B, int64_t ldb, float beta, float* C,
                      int64_t ldc, const float* bias, int epilogue, const float* aux_in, float* aux_out,
                      int64_t ld_aux, hipStream_t st, const char* who, float* colsum = nullptr,
                      int colsum_acc = 0) {
  GemmArgs g{};
  g.colsum = colsum;
  g.colsum_acc = colsum_acc;
  g.M = M; g.N = N; g.K = K;
  g.A = A; g.lda = lda; g.B = B; g.ldb = ldb;
  g.C = C; g.ldc = ldc;
  g.alpha = alpha; g.beta = beta; g.bias = bias; g.epilogue = epilogue;
  g.aux_in = aux_in; g.aux_out = aux_out; g.ld_aux = ld_aux;
  g.splits = 1;
  // not an MFMA kernel: timed with the bandwidth/latency kernels, credited
  // with its algorithmic bytes (A, B and C once each)
  HbmTimer timer("gemm_small_kernel", 4.0 * ((double)M * K + (double)K * N + (double)M * N), st);
  const int64_t outs = M * N;
  const bool wave = K > 64;
  const dim3 grid((unsigned)(wave ? (outs + 3) / 4 : (outs + 255) / 256));
#define CNHIP_SMALL(TA, TB)                                                                  \
  if (wave)                                                                                  \
    hipLaunchKernelGGL((gemm_small_wave_kernel<TA, TB>), grid, dim3(256), 0, st, g);         \
  else                                                                                       \
    hipLaunchKernelGGL((gemm_small_thread_kernel<TA, TB>), grid, dim3(256), 0, st, g);
  if (trans_a) {
    if (trans_b) { CNHIP_SMALL(true, true) } else { CNHIP_SMALL(true, false) }
  } else {
    if (trans_b) { CNHIP_SMALL(false, true) } else { CNHIP_SMALL(false, false) }
  }
#undef CNHIP_SMALL
  return check_launch(who);
}

// split-K partials of a planned GEMM: [batches][splits][M, N]
static size_t split_bytes(const Plan& plan, int64_t M, int64_t N, int64_t batches) {
  return plan.splits > 1 ? (size_t)batches * (size_t)plan.splits * (size_t)M * (size_t)N * sizeof(float) : 0;
}

size_t gemm_scratch_bytes(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, int64_t batches) {
  if (M <= 0 || N <= 0 || K < 0 || batches <= 0) return 0;
  if (gemm_is_small(M, N, K, batches, trans_a, trans_b)) return 0;
  return split_bytes(plan_gemm(trans_a, trans_b, M, N, K, batches, 64), M, N, batches);
}


static int check_spec(const GemmSpec& s, const char* who) {
  CNHIP_REQUIRE(s.M >= 0 && s.N >= 0 && s.K >= 0 && s.batches >= 0,
                "%s: negative GEMM size (M=%lld N=%lld K=%lld batch=%lld)", who, (long long)s.M,
                (long long)s.N, (long long)s.K, (long long)s.batches);
  if (s.M == 0 || s.N == 0 || s.batches == 0) return CNHIP_OK;
  CNHIP_REQUIRE(s.C != nullptr, "%s: C is NULL", who);
  CNHIP_REQUIRE(s.ldc >= s.M, "%s: ldc=%lld < M=%lld", who, (long long)s.ldc, (long long)s.M);
  if (s.K > 0) {
    CNHIP_REQUIRE(s.A && s.B, "%s: A or B is NULL", who);
    CNHIP_REQUIRE(s.lda >= (s.trans_a ? s.K : s.M), "%s: lda=%lld too small", who, (long long)s.lda);
    CNHIP_REQUIRE(s.ldb >= (s.trans_b ? s.N : s.K), "%s: ldb=%lld too small", who, (long long)s.ldb);
  }
  CNHIP_REQUIRE(s.batches <= 65535, "%s: batch count %lld exceeds 65535", who, (long long)s.batches);
  return CNHIP_OK;
}

static GemmArgs args_of(const GemmSpec& s, const Plan& plan) {
  GemmArgs g;
  g.M = s.M; g.N = s.N; g.K = s.K;
  g.A = s.A; g.lda = s.lda; g.stride_a = s.stride_a;
  g.B = s.B; g.ldb = s.ldb; g.stride_b = s.stride_b;
  g.C = s.C; g.ldc = s.ldc; g.stride_c = s.stride_c;
  g.alpha = s.alpha; g.beta = s.beta; g.bias = s.bias; g.epilogue = s.epilogue;
  g.aux_in = s.aux_in; g.aux_out = s.aux_out; g.ld_aux = s.ld_aux;
  g.vec_ok = (s.lda % 4 == 0) && (s.ldb % 4 == 0) && (s.stride_a % 4 == 0) && (s.stride_b % 4 == 0) &&
             aligned16(s.A) && aligned16(s.B);
  g.c_vec_ok = (s.ldc % 4 == 0) && (s.stride_c % 4 == 0) && aligned16(s.C);
  g.aux_vec_ok = (s.ld_aux % 4 == 0) && s.aux_in && aligned16(s.aux_in) && s.batches == 1;
  g.partial = nullptr;
  g.k_per_split = plan.kps;
  g.splits = plan.splits;
  g.colsum = nullptr;
  g.colsum_acc = 0;
  return g;
}

int column_sum(const float* in, float* out, int64_t rows, int64_t cols, int accumulate, hipStream_t st,
               const char* who);

// The fixed-order sum of a split GEMM's partials into C (with its epilogue).
static int splitk_reduce(const GemmArgs& g, int64_t batches, hipStream_t st, const char* who,
                         const ColsumJob* cs = nullptr) {
  // reads the partials (and C when beta != 0), writes C
  const double mn = (double)g.M * (double)g.N * (double)batches;
  const bool vec = g.M % 4 == 0 && g.M * g.N * batches < ((int64_t)1 << 31);
  if (vec && cs && (cs->cols + 3) / 4 < ((int64_t)1 << 30)) {
    HbmTimer timer("splitk_reduce_colsum_kernel",
                   4.0 * mn * (g.splits + 1 + (g.beta != 0.f ? 1 : 0)) +
                       4.0 * (double)cs->rows * (double)cs->cols + (cs->accumulate ? 8.0 : 4.0) * (double)cs->cols,
                   st);
    const unsigned rblocks = elementwise_grid(g.M * g.N * batches / 4, 256);
    hipLaunchKernelGGL(splitk_reduce_colsum_kernel, dim3(rblocks + (unsigned)((cs->cols + 3) / 4)), dim3(256), 0, st,
                       g, (int)batches, (int)rblocks, *cs);
    return check_launch(who);
  }
  if (cs) CNHIP_TRY(column_sum(cs->in, cs->out, cs->rows, cs->cols, cs->accumulate, st, who));
  HbmTimer timer("splitk_reduce_kernel", 4.0 * mn * (g.splits + 1 + (g.beta != 0.f ? 1 : 0)), st);
  if (vec)
    hipLaunchKernelGGL(splitk_reduce_vec_kernel, dim3(elementwise_grid(g.M * g.N * batches / 4, 256)),
                       dim3(256), 0, st, g, (int)batches);
  else
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3(elementwise_grid(g.M * g.N * batches, 256)),
                       dim3(256), 0, st, g, batches);
  return check_launch(who);
}

// One GEMM; with cs set, also those column sums (in the split-K reduce's
// launch when the plan splits).
static int gemm_spec(const GemmSpec& s, hipStream_t st, const char* who, const ColsumJob* cs = nullptr) {
  CNHIP_TRY(check_spec(s, who));
  auto sums = [&]() -> int {
    return cs ? column_sum(cs->in, cs->out, cs->rows, cs->cols, cs->accumulate, st, who) : CNHIP_OK;
  };
  if (s.M == 0 || s.N == 0 || s.batches == 0) return sums();
  if (gemm_is_small(s.M, s.N, s.K, s.batches, s.trans_a, s.trans_b)) {
    CNHIP_TRY(gemm_small(s.trans_a, s.trans_b, s.M, s.N, s.K, s.alpha, s.A, s.lda, s.B, s.ldb, s.beta, s.C,
                         s.ldc, s.bias, s.epilogue, s.aux_in, s.aux_out, s.ld_aux, st, who));
    return sums();
  }

  const Plan plan = plan_gemm(s.trans_a, s.trans_b, s.M, s.N, s.K, s.batches, 64);
  CNHIP_REQUIRE(plan.tiles < ((int64_t)1 << 30), "%s: GEMM too large", who);
  GemmArgs g = args_of(s, plan);
  if (plan.splits > 1) {
    void* ws = nullptr;
    CNHIP_TRY(scratch(st, kScratchGemm, split_bytes(plan, s.M, s.N, s.batches), &ws, who));
    g.partial = static_cast<float*>(ws);
  }
  const int status = launch_plan(plan.shape, s.trans_a, s.trans_b, g, s.batches, st, who);
  if (status != CNHIP_OK) return status;
  if (plan.splits > 1) return splitk_reduce(g, s.batches, st, who, cs);
  return sums();
}

int gemm_f32_core(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha,
                  const float* A, int64_t lda, int64_t stride_a, const float* B, int64_t ldb,
                  int64_t stride_b, float beta, float* C, int64_t ldc, int64_t stride_c,
                  int64_t batches, const float* bias, int epilogue, const float* aux_in,
                  float* aux_out, int64_t ld_aux, hipStream_t st, const char* who) {
  const GemmSpec s{trans_a, trans_b, M, N, K, alpha, A, lda, stride_a, B, ldb, stride_b, beta, C, ldc,
                   stride_c, batches, bias, epilogue, aux_in, aux_out, ld_aux};
  return gemm_spec(s, st, who);
}

// Orientation codes of the pair kernels' two GEMMs: (trans_a, trans_b, fused
// epilogue) of the first, then of the second.
#define CNHIP_PAIR_CODE(a1, b1, f1, a2, b2, f2) ((a1) << 5 | (b1) << 4 | (f1) << 3 | (a2) << 2 | (b2) << 1 | (f2))

// x (an input gradient, NT) and y (a TN weight gradient) that both plan to
// the 256 x 256 tile without split-K, in one launch of tiles_x + tiles_y
// blocks: each CU runs one such block at a time, so the launch is the two
// GEMMs' rounds back to back, and a CU whose block of x has finished starts
// a block of y while the others still store x's tiles (as separate launches,
// every CU waits for the last tile of x and for the end-of-kernel writeback).
// Each block computes exactly as in its own launch.
static int pair_xx(const GemmSpec& x, const GemmSpec& y, const Plan& px, const Plan& py, bool fx, hipStream_t st,
            const char* who, const ColsumJob* cs) {
  using C = CfgXX;
  const void* kern = nullptr;
  if (x.trans_a == 0 && x.trans_b == 1 && y.trans_a == 1 && y.trans_b == 0)
    kern = fx ? (const void*)&gemm_pair_kernel<false, true, true, true, false, false, C>
              : (const void*)&gemm_pair_kernel<false, true, false, true, false, false, C>;
  if (!kern) {
    CNHIP_TRY(gemm_spec(x, st, who));
    return gemm_spec(y, st, who, cs);
  }
  GemmArgs gx = args_of(x, px), gy = args_of(y, py);
  const int64_t nx = px.tiles * x.batches, ny = py.tiles * y.batches;
  TimingRec* rec = timing_slot(2.0 * (double)x.M * (double)x.N * (double)x.K * (double)x.batches +
                               2.0 * (double)y.M * (double)y.N * (double)y.K * (double)y.batches);
  if (rec) (void)hipEventRecord(rec->start, st);
  const int n1 = (int)nx, t1 = (int)px.tiles, b1 = (int)x.batches, t2 = (int)py.tiles, b2 = (int)y.batches;
  void* kargs[] = {&gx, &gy, const_cast<int*>(&n1), const_cast<int*>(&t1), const_cast<int*>(&b1),
                   const_cast<int*>(&t2), const_cast<int*>(&b2)};
  int status = check_hip(hipLaunchKernel(kern, dim3((unsigned)(nx + ny)), dim3(C::NT), kargs, 0, st), who);
  if (status == CNHIP_OK) status = check_launch(who);
  if (rec) (void)hipEventRecord(rec->stop, st);
  if (status != CNHIP_OK) return status;
  return cs ? column_sum(cs->in, cs->out, cs->rows, cs->cols, cs->accumulate, st, who) : CNHIP_OK;
}

// x and y in one launch when both take the 128 x 128 tile, x does not split
// K, and together they fit the chip's 512 block slots at once (y's split
// count is lowered to fit, never raised); otherwise one after the other.
// Pairs served: x an input gradient (NT, optionally with a fused epilogue)
// or a TN product, y a TN weight gradient or an NN product.
int gemm_f32_pair(const GemmSpec& x, const GemmSpec& y, hipStream_t st, const char* who, const float* cs_in,
                  float* cs_out, int64_t cs_rows, int64_t cs_cols, int cs_accumulate) {
  CNHIP_TRY(check_spec(x, who));
  CNHIP_TRY(check_spec(y, who));
  CNHIP_REQUIRE(!cs_out || (cs_rows >= 0 && cs_cols >= 0 && (cs_rows == 0 || cs_in)), "%s: bad column-sum operands",
                who);
  const bool sums = cs_out && cs_cols > 0;
  const ColsumJob cs{cs_in, cs_out, cs_rows, cs_cols, cs_accumulate,
                     (cs_rows % 4 == 0) && aligned16(cs_in) ? 1 : 0};
  auto apart = [&]() -> int {
    CNHIP_TRY(gemm_spec(x, st, who));
    return gemm_spec(y, st, who, sums ? &cs : nullptr);
  };
  auto big = [](const GemmSpec& s) {
    return s.M > 0 && s.N > 0 && s.K > 0 && s.batches > 0 &&
           !gemm_is_small(s.M, s.N, s.K, s.batches, s.trans_a, s.trans_b);
  };
  if (!big(x) || !big(y)) return apart();
  const Plan px = plan_gemm(x.trans_a, x.trans_b, x.M, x.N, x.K, x.batches, 64);
  Plan py = plan_gemm(y.trans_a, y.trans_b, y.M, y.N, y.K, y.batches, 64);
  const bool fx = !x.trans_a && x.epilogue >= EPI_GELU;
  if (px.shape == Shape::XX && py.shape == Shape::XX && px.splits == 1 && py.splits == 1)
    return pair_xx(x, y, px, py, fx, st, who, sums ? &cs : nullptr);
  if (px.shape != Shape::M || py.shape != Shape::M || px.splits != 1) return apart();
  constexpr int64_t kSlots = 512;  // 2 blocks of 512 threads per CU, 256 CUs
  const int64_t nx = px.tiles * x.batches, ty = py.tiles * y.batches;
  if (nx + ty > kSlots) return apart();
  if (nx + ty * py.splits > kSlots) {
    const int fit = (int)((kSlots - nx) / ty);
    int64_t kps = (y.K + fit - 1) / fit;
    kps = ((kps + KQ - 1) / KQ) * KQ;
    py.kps = kps;
    py.splits = (int)((y.K + kps - 1) / kps);
  }
  const bool fy = !y.trans_a && y.epilogue >= EPI_GELU;
  const int code = CNHIP_PAIR_CODE(x.trans_a, x.trans_b, fx ? 1 : 0, y.trans_a, y.trans_b, fy && py.splits == 1 ? 1 : 0);
  using C = CfgM;
  const void* kern = nullptr;
  switch (code) {
    case CNHIP_PAIR_CODE(0, 1, 1, 1, 0, 0): kern = (const void*)&gemm_pair_kernel<false, true, true, true, false, false, C>; break;
    case CNHIP_PAIR_CODE(0, 1, 0, 1, 0, 0): kern = (const void*)&gemm_pair_kernel<false, true, false, true, false, false, C>; break;
    case CNHIP_PAIR_CODE(1, 0, 0, 0, 0, 0): kern = (const void*)&gemm_pair_kernel<true, false, false, false, false, false, C>; break;
    default: return apart();
  }
  GemmArgs gx = args_of(x, px), gy = args_of(y, py);
  if (py.splits > 1) {
    void* ws = nullptr;
    CNHIP_TRY(scratch(st, kScratchGemm, split_bytes(py, y.M, y.N, y.batches), &ws, who));
    gy.partial = static_cast<float*>(ws);
  }
  const int64_t ny = ty * py.splits;
  TimingRec* rec = timing_slot(2.0 * (double)x.M * (double)x.N * (double)x.K * (double)x.batches +
                               2.0 * (double)y.M * (double)y.N * (double)y.K * (double)y.batches);
  if (rec) (void)hipEventRecord(rec->start, st);
  const int n1 = (int)nx, t1 = (int)px.tiles, b1 = (int)x.batches, t2 = (int)py.tiles, b2 = (int)y.batches;
  void* kargs[] = {&gx, &gy, const_cast<int*>(&n1), const_cast<int*>(&t1), const_cast<int*>(&b1),
                   const_cast<int*>(&t2), const_cast<int*>(&b2)};
  int status = check_hip(hipLaunchKernel(kern, dim3((unsigned)(nx + ny)), dim3(C::NT), kargs, 0, st), who);
  if (status == CNHIP_OK) status = check_launch(who);
  if (rec) (void)hipEventRecord(rec->stop, st);
  if (status != CNHIP_OK) return status;
  // the column sums ride in the split reduce's launch when there is one
  if (py.splits > 1) return splitk_reduce(gy, y.batches, st, who, sums ? &cs : nullptr);
  return sums ? column_sum(cs_in, cs_out, cs_rows, cs_cols, cs_accumulate, st, who) : CNHIP_OK;
}
#undef CNHIP_PAIR_CODE

int gemm_f32(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha,
             const float* A, int64_t lda, const float* B, int64_t ldb, float beta, float* C,
             int64_t ldc, const float* bias, int epilogue, hipStream_t st, const char* who) {
  return gemm_f32_batched(trans_a, trans_b, M, N, K, alpha, A, lda, 0, B, ldb, 0, beta, C, ldc, 0,
                          1, bias, epilogue, st, who);
}

int linear_wgrad_small(const float* X, const float* dY, float* dW, float* db, int64_t batch,
                       int64_t in_features, int64_t out_features, int accumulate, hipStream_t st,
                       const char* who, bool* done) {
  *done = false;
  if (!gemm_is_small(in_features, out_features, batch, 1, 1, 0)) return CNHIP_OK;
  CNHIP_REQUIRE(X && dY && dW, "%s: NULL pointer", who);
  *done = true;
  return gemm_small(1, 0, in_features, out_features, batch, 1.f, X, batch, dY, batch,
                    accumulate ? 1.f : 0.f, dW, in_features, nullptr, CNHIP_EPI_NONE, nullptr, nullptr, 0,
                    st, who, db, accumulate);
}

// A Linear layer's weight gradient with its bias sums and its input gradient
// in one launch when both are small GEMMs (a small head: config 4's 512 -> 1
// over 128 samples): the same kernels' blocks as linear_wgrad_small's launch
// followed by the dX launch, so the same bits.
int linear_backward_small_pair(const float* X, const float* W, const float* dY, float* dW, float* db, float* dX,
                               int64_t batch, int64_t in_features, int64_t out_features, int accumulate,
                               hipStream_t st, const char* who, bool* done) {
  *done = false;
  if (batch <= 0 || !dX || !gemm_is_small(in_features, out_features, batch, 1, 1, 0) ||
      !gemm_is_small(batch, in_features, out_features, 1, 0, 1))
    return CNHIP_OK;
  CNHIP_REQUIRE(X && W && dY && dW, "%s: NULL pointer", who);
  *done = true;
  auto args = [](int64_t M, int64_t N, int64_t K, const float* A, int64_t lda, const float* B, int64_t ldb,
                 float beta, float* C, int64_t ldc, float* colsum, int colsum_acc) {
    GemmArgs g{};
    g.colsum = colsum;
    g.colsum_acc = colsum_acc;
    g.M = M; g.N = N; g.K = K;
    g.A = A; g.lda = lda; g.B = B; g.ldb = ldb;
    g.C = C; g.ldc = ldc;
    g.alpha = 1.f; g.beta = beta; g.bias = nullptr; g.epilogue = CNHIP_EPI_NONE;
    g.splits = 1;
    return g;
  };
  // dW[I,O] (+)= X^T dY with db (+)= the column sums of dY; dX[B,I] = dY W^T
  const GemmArgs gw = args(in_features, out_features, batch, X, batch, dY, batch, accumulate ? 1.f : 0.f, dW,
                           in_features, db, accumulate);
  const GemmArgs gx = args(batch, in_features, out_features, dY, batch, W, in_features, 0.f, dX, batch, nullptr, 0);
  const bool w1 = batch > 64, w2 = out_features > 64;  // as gemm_small chooses
  const int64_t o1 = in_features * out_features, o2 = batch * in_features;
  const int64_t n1 = w1 ? (o1 + 3) / 4 : (o1 + 255) / 256, n2 = w2 ? (o2 + 3) / 4 : (o2 + 255) / 256;
  HbmTimer timer("gemm_small_kernel",
                 4.0 * ((double)in_features * batch + (double)batch * out_features + (double)o1) +
                     4.0 * ((double)batch * out_features + (double)out_features * in_features + (double)o2),
                 st);
  const dim3 grid((unsigned)(n1 + n2));
  if (w1 && w2) hipLaunchKernelGGL((gemm_small_pair_kernel<true, true>), grid, dim3(256), 0, st, gw, gx, n1);
  else if (w1) hipLaunchKernelGGL((gemm_small_pair_kernel<true, false>), grid, dim3(256), 0, st, gw, gx, n1);
  else if (w2) hipLaunchKernelGGL((gemm_small_pair_kernel<false, true>), grid, dim3(256), 0, st, gw, gx, n1);
  else hipLaunchKernelGGL((gemm_small_pair_kernel<false, false>), grid, dim3(256), 0, st, gw, gx, n1);
  return check_launch(who);
}

int gemm_f32_act(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, const float* A,
                 int64_t lda, const float* B, int64_t ldb, float* C, int64_t ldc, const float* bias,
                 int epilogue, const float* aux_in, float* aux_out, int64_t ld_aux, hipStream_t st,
                 const char* who) {
  const bool needs_in = epilogue == EPI_DRELU || epilogue == EPI_DGELU || epilogue == EPI_ADD;
  CNHIP_REQUIRE(trans_a == 0 || epilogue < EPI_GELU, "%s: fused activations need trans_a == 0", who);
  CNHIP_REQUIRE(epilogue == CNHIP_EPI_NONE || epilogue == CNHIP_EPI_RELU || epilogue == EPI_GELU ||
                    needs_in,
                "%s: bad epilogue %d", who, epilogue);
  CNHIP_REQUIRE((epilogue != EPI_GELU || aux_out) && (!needs_in || aux_in) &&
                    (!(aux_in || aux_out) || ld_aux >= M),
                "%s: fused activation needs its [M,N] side tensor (ld >= M)", who);
  return gemm_f32_core(trans_a, trans_b, M, N, K, 1.f, A, lda, 0, B, ldb, 0, 0.f, C, ldc, 0, 1, bias,
                       epilogue, aux_in, aux_out, ld_aux, st, who);
}


}  // namespace cnhip

extern "C" int cnhip_gemm_f32(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K,
                              float alpha, const float* A, int64_t lda, const float* B,
                              int64_t ldb, float beta, float* C, int64_t ldc, const float* bias,
                              int epilogue, cnhip_stream_t stream) {
  return cnhip::gemm_f32(trans_a, trans_b, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, bias,
                         epilogue, cnhip::as_stream(stream), "cnhip_gemm_f32");
}

extern "C" int cnhip_gemm_f32_batched(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K,
                                      float alpha, const float* A, int64_t lda, int64_t stride_a,
                                      const float* B, int64_t ldb, int64_t stride_b, float beta,
                                      float* C, int64_t ldc, int64_t stride_c, int64_t batch_count,
                                      cnhip_stream_t stream) {
  return cnhip::gemm_f32_batched(trans_a, trans_b, M, N, K, alpha, A, lda, stride_a, B, ldb,
                                 stride_b, beta, C, ldc, stride_c, batch_count, nullptr,
                                 CNHIP_EPI_NONE, cnhip::as_stream(stream),
                                 "cnhip_gemm_f32_batched");
}

extern "C" int cnhip_gemm_timing_enable(int on) {
  cnhip::g_timing.on = on != 0;
  cnhip::g_timing.used = 0;
  return CNHIP_OK;
}

extern "C" int cnhip_gemm_timing_read(int64_t* launches, double* total_ms, double* total_flops) {
  CNHIP_REQUIRE(launches && total_ms && total_flops, "cnhip_gemm_timing_read: NULL argument");
  cnhip::Timing& t = cnhip::g_timing;
  double ms = 0.0, fl = 0.0;
  for (size_t i = 0; i < t.used; ++i) {
    float e = 0.f;
    CNHIP_TRY(cnhip::check_hip(hipEventSynchronize(t.pool[i].stop), "cnhip_gemm_timing_read"));
    CNHIP_TRY(cnhip::check_hip(hipEventElapsedTime(&e, t.pool[i].start, t.pool[i].stop),
                               "cnhip_gemm_timing_read"));
    ms += e;
    fl += t.pool[i].flops;
  }
  *launches = (int64_t)t.used;
  *total_ms = ms;
  *total_flops = fl;
  return CNHIP_OK;
}

extern "C" int cnhip_hbm_timing_enable(int on) {
  cnhip::g_hbm_timing.on = on != 0;
  cnhip::g_hbm_timing.used = 0;
  return CNHIP_OK;
}

extern "C" int cnhip_hbm_timing_read(cnhip_kernel_timing* rows, int max_rows, int* n_rows) {
  const char* who = "cnhip_hbm_timing_read";
  CNHIP_REQUIRE(n_rows && (rows || max_rows == 0) && max_rows >= 0, "%s: bad arguments", who);
  cnhip::Timing& t = cnhip::g_hbm_timing;
  std::vector<cnhip_kernel_timing> agg;  // per kernel name, first-seen order
  for (size_t i = 0; i < t.used; ++i) {
    const cnhip::TimingRec& r = t.pool[i];
    float e = 0.f;
    CNHIP_TRY(cnhip::check_hip(hipEventSynchronize(r.stop), who));
    CNHIP_TRY(cnhip::check_hip(hipEventElapsedTime(&e, r.start, r.stop), who));
    size_t k = 0;
    while (k < agg.size() && std::strcmp(agg[k].kernel, r.kernel) != 0) ++k;
    if (k == agg.size()) agg.push_back(cnhip_kernel_timing{r.kernel, 0, 0.0, 0.0});
    agg[k].launches += 1;
    agg[k].total_ms += e;
    agg[k].total_bytes += r.bytes;
  }
  for (size_t k = 0; k < agg.size() && (int)k < max_rows; ++k) rows[k] = agg[k];
  *n_rows = (int)agg.size();
  return CNHIP_OK;
}
