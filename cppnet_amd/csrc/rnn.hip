// LSTM and GRU forward / backward-through-time on MI355X.
//
// ref: LSTM::forward/backward src/CppNet/layers/lstm.cpp:63-253,
//      GRU::forward/backward  src/CppNet/layers/gru.cpp:56-297,
//      lstm_cell.cu:21-114, gru_cell.cu:20-140 (reference gpu gate kernels,
//      driven with per-timestep host round trips of every cache).
//
// Layout: X [B,S,I], Y [B,S,H] ColMajor, i.e. [B*S, I] / [B*S, H] matrices
// whose row index is n + B*t, so timestep t is the row block [B*t, B*t+B).
// The reference computes x_t W_ih and every weight gradient inside its time
// loop.  Here the parts that do not depend on the recurrence run once over
// all B*S rows as large MFMA GEMMs:
//   forward : G = X W_ih (all steps), then per step one launch of
//             h_{t-1} W_hh with the LSTM cell in its epilogue
//   backward: per step one launch of dh_t = dY_t + dG_{t+1} W_hh^T with the
//             cell backward in its epilogue; afterwards dW_ih = X^T dG,
//             dW_hh = Y_{t-1}^T dG, db = colsum dG, dX = dG W_ih^T, each a
//             single GEMM over all B*S rows.
// The cell kernels fuse every elementwise gate computation of a step into one
// pass (one thread per (n, d); n fastest for coalescing) and evaluate the
// reference expressions in the reference's operation order.
#include <hip/hip_runtime.h>

#include <cmath>

#include "common.hpp"
#include "mfma_kpack.hpp"

namespace cnhip {

int gemm_f32(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha,
             const float* A, int64_t lda, const float* B, int64_t ldb, float beta, float* C,
             int64_t ldc, const float* bias, int epilogue, hipStream_t st, const char* who);
int column_sum(const float* in, float* out, int64_t rows, int64_t cols, int accumulate,
               hipStream_t st, const char* who);
int gemm_f32_core(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha,
                  const float* A, int64_t lda, int64_t stride_a, const float* B, int64_t ldb,
                  int64_t stride_b, float beta, float* C, int64_t ldc, int64_t stride_c,
                  int64_t batches, const float* bias, int epilogue, const float* aux_in,
                  float* aux_out, int64_t ld_aux, hipStream_t st, const char* who);
int fill_bytes(void* dst, int value, size_t bytes, hipStream_t stream, const char* where);
constexpr int EPI_TANH = 6;  // GEMM epilogue C = tanh(v) (gemm_f32.hip)

namespace {

__device__ __forceinline__ float sigm(float x) { return 1.0f / (1.0f + expf(-x)); }

// ---------------------------------------------------------------- LSTM cell
// Step t = 0 (h_0 = c_0 = 0, so no recurrent term): the rows of step 0 of
// gates hold x W_ih and are overwritten with the activations i, f, g, o
// (lstm.cpp:115-134); later steps run lstm_step_fwd_kernel.
__global__ void __launch_bounds__(256) lstm_cell_fwd0_kernel(float* __restrict__ gates,
                                                             const float* __restrict__ bias,
                                                             float* __restrict__ c,
                                                             float* __restrict__ tanh_c,
                                                             float* __restrict__ Y, int64_t B,
                                                             int64_t S, int64_t H) {
  const int64_t BS = B * S;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= B * H) return;
  const int64_t n = e % B, d = e / B, row = n;
  float* g = gates + row;
  const float ig = sigm(g[BS * d] + bias[d]);
  const float fg = sigm(g[BS * (d + H)] + bias[d + H]);
  const float gg = tanhf(g[BS * (d + 2 * H)] + bias[d + 2 * H]);
  const float og = sigm(g[BS * (d + 3 * H)] + bias[d + 3 * H]);
  const float ct = fg * 0.0f + ig * gg;
  const float tc = tanhf(ct);
  g[BS * d] = ig;
  g[BS * (d + H)] = fg;
  g[BS * (d + 2 * H)] = gg;
  g[BS * (d + 3 * H)] = og;
  c[row + BS * d] = ct;
  tanh_c[row + BS * d] = tc;
  Y[row + BS * d] = og * tc;
}

// One forward timestep t >= 1 in one launch: the recurrent GEMM
// h_{t-1} W_hh for a tile of 32 samples x (8 hidden units x 4 gates) and
// the cell update of those 256 (sample, unit) pairs in its epilogue.  The 4
// gate columns of a unit sit in one tile, so no other block's result is
// needed; the k-tile (64) is split over 4 wave groups whose partial sums are
// added in a fixed order.  256 blocks cover B = 128, H = 512.
using kp::f32x4;
using LstmFwdCfg = kp::Cfg<1, 1, 1, 1, 16, 4>;
constexpr int kLstmUnits = 8;  // hidden units per tile

template <class LstmCfg, bool FAST>
struct LstmFwdStage {
  using OA = kp::Operand<false, 32, LstmCfg::NT, LstmCfg::KT>;  // h(b, k) = Y[b + B(t-1) + BS k]
  using OB = kp::Operand<true, 32, LstmCfg::NT, LstmCfg::KT>;   // W_hh(k, col(n)), k-contiguous
  const float* A;  // Y + B*(t-1)
  const float* W;
  int64_t BS, B, H, b0, j0;
  f32x4 ra[2][OA::REGS], rb[2][OB::REGS];

  __device__ LstmFwdStage(const float* A_, const float* W_, int64_t BS_, int64_t B_, int64_t H_,
                          int64_t b0_, int64_t j0_)
      : A(A_), W(W_), BS(BS_), B(B_), H(H_), b0(b0_), j0(j0_) {}

  template <int S>
  __device__ __forceinline__ void load(int t) {
    const int64_t k0 = (int64_t)t * LstmCfg::KT;
    OA::template load<FAST>(A, BS, b0, k0, B, H, ra[S]);
#pragma unroll
    for (int p = 0; p < OB::PER; ++p) {
      int r, k;
      if (!OB::origin(p, r, k)) break;
      // tile column r = gate * 8 + unit: W_hh column gate*H + j0 + unit
      const int64_t j = j0 + r % kLstmUnits, gk = k0 + k;
      const float* col = W + H * ((r / kLstmUnits) * H + j);
      if (FAST) {
        rb[S][p] = *reinterpret_cast<const f32x4*>(col + gk);
      } else {
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (j < H && gk + e < H) ? col[gk + e] : 0.f;
        rb[S][p] = v;
      }
    }
  }
  template <int S>
  __device__ __forceinline__ void store(float* buf) {
    OA::store(buf, ra[S]);
    OB::store(buf + OA::FLOATS, rb[S]);
  }
};

template <class LstmCfg, bool FAST>
__global__ void __launch_bounds__(LstmCfg::NT) lstm_step_fwd_kernel(
    float* __restrict__ gates, const float* __restrict__ bias, float* __restrict__ c,
    float* __restrict__ tanh_c, float* __restrict__ Y, const float* __restrict__ W_hh, int64_t B,
    int64_t S, int64_t H, int64_t t) {
  constexpr int FLOATS = 2 * kp::stage_floats<LstmFwdStage<LstmCfg, FAST>>();
  static_assert((LstmCfg::WGK - 1) * 1024 <= FLOATS, "reduce_wgk needs more LDS");
  __shared__ __align__(16) float lds[FLOATS];
  __shared__ float tile[32 * 33];  // [col][row], padded
  const int64_t BS = B * S;
  const int nbt = (int)((B + 31) / 32);
  const int64_t b0 = (int64_t)(blockIdx.x % nbt) * 32;
  const int64_t j0 = (int64_t)(blockIdx.x / nbt) * kLstmUnits;
  kp::f32x16 acc[1][1];
  kp::zero_acc<LstmCfg>(acc);
  LstmFwdStage<LstmCfg, FAST> s(Y + B * (t - 1), W_hh, BS, B, H, b0, j0);
  kp::pipeline<LstmCfg>((int)((H + LstmCfg::KT - 1) / LstmCfg::KT), lds, s, acc);
  kp::reduce_wgk<LstmCfg>(lds, acc);
  kp::for_each_acc_run<LstmCfg>(acc, [&](int ml, int nl, const kp::f32x4& v) {
#pragma unroll
    for (int e = 0; e < 4; ++e) tile[(ml + e) + 33 * nl] = v[e];
  });
  __syncthreads();
  // thread -> (sample, unit): the cell of lstm_cell_fwd0_kernel with the
  // recurrent term h W_hh taken from the tile
  static_assert(LstmCfg::NT >= 32 * kLstmUnits, "one thread per (sample, unit)");
  const int bl = threadIdx.x % 32, u = threadIdx.x / 32;
  if (u >= kLstmUnits) return;
  const int64_t n = b0 + bl, d = j0 + u;
  if (n >= B || d >= H) return;
  const int64_t row = n + B * t;
  float* g = gates + row;
  auto pre = [&](int gate, int64_t j) { return tile[bl + 33 * (gate * kLstmUnits + u)] + g[BS * j]; };
  const float ig = sigm(pre(0, d) + bias[d]);
  const float fg = sigm(pre(1, d + H) + bias[d + H]);
  const float gg = tanhf(pre(2, d + 2 * H) + bias[d + 2 * H]);
  const float og = sigm(pre(3, d + 3 * H) + bias[d + 3 * H]);
  const float cprev = c[row - B + BS * d];
  const float ct = fg * cprev + ig * gg;
  const float tc = tanhf(ct);
  g[BS * d] = ig;
  g[BS * (d + H)] = fg;
  g[BS * (d + 2 * H)] = gg;
  g[BS * (d + 3 * H)] = og;
  c[row + BS * d] = ct;
  tanh_c[row + BS * d] = tc;
  Y[row + BS * d] = og * tc;
}

// lstm.cpp:184-219, 247-249, the last step t = S-1: dh = dY (no later step)
// and dc starts from 0; dc_buf [B, H] (ld B) receives dc * f for step t-1.
// Earlier steps run lstm_step_bwd_kernel.
__global__ void __launch_bounds__(256) lstm_cell_bwd_last_kernel(
    const float* __restrict__ gates, const float* __restrict__ c, const float* __restrict__ tanh_c,
    const float* __restrict__ dY, float* __restrict__ dc_buf, float* __restrict__ dG, int64_t B,
    int64_t S, int64_t H) {
  const int64_t BS = B * S, t = S - 1;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= B * H) return;
  const int64_t n = e % B, d = e / B, row = n + B * t;
  const float ig = gates[row + BS * d], fg = gates[row + BS * (d + H)];
  const float gg = gates[row + BS * (d + 2 * H)], og = gates[row + BS * (d + 3 * H)];
  const float tc = tanh_c[row + BS * d];
  const float dh = dY[row + BS * d];
  const float dc = dh * og * (1.0f - tc * tc) + 0.0f;
  const float cprev = t > 0 ? c[row - B + BS * d] : 0.0f;
  dG[row + BS * d] = dc * gg * ig * (1.0f - ig);
  dG[row + BS * (d + H)] = dc * cprev * fg * (1.0f - fg);
  dG[row + BS * (d + 2 * H)] = dc * ig * (1.0f - gg * gg);
  dG[row + BS * (d + 3 * H)] = dh * tc * og * (1.0f - og);
  dc_buf[e] = dc * fg;
}

// One backward timestep t <= S-2 in one launch: dh_t = dY_t + dG_{t+1} W_hh^T
// for a tile of 16 samples x 16 hidden units (K = 4H split over the wave
// groups of the block, added in a fixed order), then lstm_cell_bwd_last_kernel's
// arithmetic for those 256 (sample, unit) pairs in the epilogue.  16 x 16
// tiles give 256 blocks at B = 128, H = 512.
using LstmBwdCfgDefault = kp::Cfg16<1, 1, 1, 1, 32, 8>;  // fastest of a measured sweep

template <class LstmBwdCfg, bool FAST>
struct LstmBwdStage {
  using OA = kp::Operand<false, 16, LstmBwdCfg::NT, LstmBwdCfg::KT>;  // dG(b, k) = dG[b + BS k]
  using OB = kp::Operand<false, 16, LstmBwdCfg::NT, LstmBwdCfg::KT>;  // W_hh^T(j, k) = W_hh[j + H k]
  const float* A;  // dG + B*(t+1)
  const float* W;
  int64_t BS, B, H, b0, j0;
  f32x4 ra[2][OA::REGS], rb[2][OB::REGS];

  __device__ LstmBwdStage(const float* A_, const float* W_, int64_t BS_, int64_t B_, int64_t H_,
                          int64_t b0_, int64_t j0_)
      : A(A_), W(W_), BS(BS_), B(B_), H(H_), b0(b0_), j0(j0_) {}

  template <int S>
  __device__ __forceinline__ void load(int t) {
    const int64_t k0 = (int64_t)t * LstmBwdCfg::KT;
    OA::template load<FAST>(A, BS, b0, k0, B, 4 * H, ra[S]);
    OB::template load<FAST>(W, H, j0, k0, H, 4 * H, rb[S]);
  }
  template <int S>
  __device__ __forceinline__ void store(float* buf) {
    OA::store(buf, ra[S]);
    OB::store(buf + OA::FLOATS, rb[S]);
  }
};

template <class LstmBwdCfg, bool FAST>
__global__ void __launch_bounds__(LstmBwdCfg::NT) lstm_step_bwd_kernel(
    const float* __restrict__ gates, const float* __restrict__ c, const float* __restrict__ tanh_c,
    const float* __restrict__ dY, const float* __restrict__ W_hh, float* __restrict__ dc_buf,
    float* __restrict__ dG, int64_t B, int64_t S, int64_t H, int64_t t) {
  constexpr int FLOATS = 2 * kp::stage_floats<LstmBwdStage<LstmBwdCfg, FAST>>();
  static_assert((LstmBwdCfg::WGK - 1) * 4 * 64 <= FLOATS, "reduce_wgk16 needs more LDS");
  __shared__ __align__(16) float lds[FLOATS];
  __shared__ float tile[16 * 17];  // [unit][sample], padded
  const int64_t BS = B * S;
  const int nbt = (int)((B + 15) / 16);
  const int64_t b0 = (int64_t)(blockIdx.x % nbt) * 16;
  const int64_t j0 = (int64_t)(blockIdx.x / nbt) * 16;
  f32x4 acc[1][1];
  kp::zero_acc16<LstmBwdCfg>(acc);
  LstmBwdStage<LstmBwdCfg, FAST> s(dG + B * (t + 1), W_hh, BS, B, H, b0, j0);
  kp::pipeline<LstmBwdCfg>((int)((4 * H + LstmBwdCfg::KT - 1) / LstmBwdCfg::KT), lds, s, acc);
  kp::reduce_wgk16<LstmBwdCfg>(lds, acc);
  kp::for_each_acc_run16<LstmBwdCfg>(acc, [&](int ml, int nl, const f32x4& v) {
#pragma unroll
    for (int e = 0; e < 4; ++e) tile[(ml + e) + 17 * nl] = v[e];
  });
  __syncthreads();
  static_assert(LstmBwdCfg::NT >= 256, "one thread per (sample, unit)");
  const int bl = threadIdx.x % 16, jl = threadIdx.x / 16;
  if (jl >= 16) return;
  const int64_t n = b0 + bl, d = j0 + jl;
  if (n >= B || d >= H) return;
  const int64_t e = n + B * d, row = n + B * t;
  const float ig = gates[row + BS * d], fg = gates[row + BS * (d + H)];
  const float gg = gates[row + BS * (d + 2 * H)], og = gates[row + BS * (d + 3 * H)];
  const float tc = tanh_c[row + BS * d];
  const float dh = dY[row + BS * d] + tile[bl + 17 * jl];
  const float dc = dh * og * (1.0f - tc * tc) + dc_buf[e];
  const float cprev = t > 0 ? c[row - B + BS * d] : 0.0f;
  dG[row + BS * d] = dc * gg * ig * (1.0f - ig);
  dG[row + BS * (d + H)] = dc * cprev * fg * (1.0f - fg);
  dG[row + BS * (d + 2 * H)] = dc * ig * (1.0f - gg * gg);
  dG[row + BS * (d + 3 * H)] = dh * tc * og * (1.0f - og);
  dc_buf[e] = dc * fg;
}

// ---------------------------------------------------------------- GRU cells
// gru.cpp:102-109: z, r from x W_ih + h W_hh (+ b); rh = r * h_prev.
// hz: [B, 2H] dense = h_{t-1} W_hh[:, 0:2H] (ignored at t = 0, where h = 0).
__global__ void __launch_bounds__(256) gru_zr_kernel(float* __restrict__ gates,
                                                     const float* __restrict__ hz,
                                                     const float* __restrict__ bias,
                                                     const float* __restrict__ Y,
                                                     float* __restrict__ rh, int64_t B, int64_t S,
                                                     int64_t H, int64_t t) {
  const int64_t BS = B * S;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= B * H) return;
  const int64_t n = e % B, d = e / B, row = n + B * t;
  const float hzz = t > 0 ? hz[n + B * d] : 0.0f;
  const float hzr = t > 0 ? hz[n + B * (d + H)] : 0.0f;
  const float zg = sigm((gates[row + BS * d] + hzz) + bias[d]);
  const float rg = sigm((gates[row + BS * (d + H)] + hzr) + bias[d + H]);
  const float hp = t > 0 ? Y[row - B + BS * d] : 0.0f;
  gates[row + BS * d] = zg;
  gates[row + BS * (d + H)] = rg;
  rh[row + BS * d] = rg * hp;
}

// gru.cpp:120-133: n = tanh(x W_in + rh W_hn + b_n), h = (1-z) n + z h_prev.
__global__ void __launch_bounds__(256) gru_n_kernel(float* __restrict__ gates,
                                                    const float* __restrict__ proj,
                                                    const float* __restrict__ bias,
                                                    float* __restrict__ Y, int64_t B, int64_t S,
                                                    int64_t H, int64_t t) {
  const int64_t BS = B * S;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= B * H) return;
  const int64_t n = e % B, d = e / B, row = n + B * t;
  const float zg = gates[row + BS * d];
  const float nc = tanhf((gates[row + BS * (d + 2 * H)] + proj[n + B * d]) + bias[d + 2 * H]);
  const float hp = t > 0 ? Y[row - B + BS * d] : 0.0f;
  gates[row + BS * (d + 2 * H)] = nc;
  Y[row + BS * d] = (1.0f - zg) * nc + zg * hp;
}

// gru.cpp:188-209.  dh: [B,H] dense, holds dh_next on entry (ignored when
// first) and dh_prev's direct part (dh * z) on exit.
__global__ void __launch_bounds__(256) gru_bwd_a_kernel(const float* __restrict__ gates,
                                                        const float* __restrict__ Y,
                                                        const float* __restrict__ dY,
                                                        float* __restrict__ dh,
                                                        float* __restrict__ dG, int64_t B,
                                                        int64_t S, int64_t H, int64_t t,
                                                        int first) {
  const int64_t BS = B * S;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= B * H) return;
  const int64_t n = e % B, d = e / B, row = n + B * t;
  const float zg = gates[row + BS * d], nc = gates[row + BS * (d + 2 * H)];
  const float hp = t > 0 ? Y[row - B + BS * d] : 0.0f;
  const float dhv = dY[row + BS * d] + (first ? 0.0f : dh[e]);
  const float dn = dhv * (1.0f - zg);
  const float dz = dhv * (hp - nc);
  dG[row + BS * d] = dz * zg * (1.0f - zg);
  dG[row + BS * (d + 2 * H)] = dn * (1.0f - nc * nc);
  dh[e] = dhv * zg;
}

// gru.cpp:214-225: with d_rh = dn_raw W_hn^T, dr_raw and dh_prev += d_rh * r.
__global__ void __launch_bounds__(256) gru_bwd_b_kernel(const float* __restrict__ gates,
                                                        const float* __restrict__ Y,
                                                        const float* __restrict__ d_rh,
                                                        float* __restrict__ dh,
                                                        float* __restrict__ dG, int64_t B,
                                                        int64_t S, int64_t H, int64_t t) {
  const int64_t BS = B * S;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= B * H) return;
  const int64_t n = e % B, d = e / B, row = n + B * t;
  const float rg = gates[row + BS * (d + H)];
  const float hp = t > 0 ? Y[row - B + BS * d] : 0.0f;
  const float dr = d_rh[e] * hp;
  dG[row + BS * (d + H)] = dr * rg * (1.0f - rg);
  dh[e] += d_rh[e] * rg;
}

// out[B, D] = Y[:, t, :]  /  Y = 0 except Y[:, t, :] = in
__global__ void __launch_bounds__(256) seq_select_kernel(const float* __restrict__ Y,
                                                         float* __restrict__ out, int64_t B,
                                                         int64_t S, int64_t D, int64_t t) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= B * D) return;
  const int64_t n = e % B, d = e / B;
  out[e] = Y[n + B * t + B * S * d];
}

__global__ void __launch_bounds__(256) seq_scatter_kernel(const float* __restrict__ in,
                                                          float* __restrict__ Y, int64_t B,
                                                          int64_t S, int64_t D, int64_t t) {
  const int64_t total = B * S * D;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = i % B, s = (i / B) % S, d = i / (B * S);
    Y[i] = s == t ? in[n + B * d] : 0.0f;
  }
}

unsigned cell_grid(int64_t B, int64_t H) { return (unsigned)((B * H + 255) / 256); }

// ---------------------------------------------------------------- Elman RNN
// rnn.cpp:48-100: step 0 has no recurrent term (h_0 = 0): its rows of Y hold
// x_0 W_ih and become tanh(x_0 W_ih + b).
__global__ void __launch_bounds__(256) rnn_step0_kernel(float* __restrict__ Y, const float* __restrict__ b,
                                                        int64_t B, int64_t BS, int64_t H) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= B * H) return;
  const int64_t n = e % B, d = e / B;
  float* y = Y + n + BS * d;
  *y = tanhf(*y + b[d]);
}
// rnn.cpp:118-131: dtanh_t = (dY_t + dh_next) * (1 - h_t^2) into dT's rows of
// step t (dh_next == nullptr at the last step: dh_next is zero there).
__global__ void __launch_bounds__(256) rnn_bwd_cell_kernel(const float* __restrict__ dY,
                                                           const float* __restrict__ Y,
                                                           const float* __restrict__ dh_next,
                                                           float* __restrict__ dT, int64_t B, int64_t BS,
                                                           int64_t H, int64_t t) {
#pragma clang fp contract(off)
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= B * H) return;
  const int64_t n = e % B, d = e / B, i = n + B * t + BS * d;
  const float dh = dh_next ? dY[i] + dh_next[n + B * d] : dY[i];
  const float h = Y[i];
  dT[i] = dh * (1.0f - h * h);
}

// Per-step launches of the fused LSTM kernels for steps t = 1 .. S-1
// (forward) and t = S-2 .. 0 (backward), each timed like a GEMM (2*B*4H*H
// flops) for the per-launch roofline.
template <class Cfg>
int lstm_fwd_steps(float* gates, const float* b, float* c, float* tanh_c, float* Y,
                   const float* W_hh, int64_t B, int64_t S, int64_t H, hipStream_t st,
                   const char* who) {
  const int64_t nbt = (B + 31) / 32, nbu = (H + kLstmUnits - 1) / kLstmUnits;
  CNHIP_REQUIRE(nbt * nbu < ((int64_t)1 << 31), "%s: too many tiles", who);
  // FAST: full tiles, whole k-tiles, 16-byte aligned rows of Y and W_hh
  const bool fast = B % 32 == 0 && H % Cfg::KT == 0 && H % kLstmUnits == 0 && (B * S) % 4 == 0 &&
                    aligned16(Y) && aligned16(W_hh);
  const auto kern = fast ? &lstm_step_fwd_kernel<Cfg, true> : &lstm_step_fwd_kernel<Cfg, false>;
  for (int64_t t = 1; t < S; ++t) {
    TimingRec* rec = timing_slot(2.0 * B * 4 * H * H);
    if (rec) (void)hipEventRecord(rec->start, st);
    hipLaunchKernelGGL(kern, dim3((unsigned)(nbt * nbu)), dim3(Cfg::NT), 0, st, gates, b, c, tanh_c,
                       Y, W_hh, B, S, H, t);
    CNHIP_TRY(check_launch(who));
    if (rec) (void)hipEventRecord(rec->stop, st);
  }
  return CNHIP_OK;
}

template <class Cfg>
int lstm_bwd_steps(const float* gates, const float* c, const float* tanh_c, const float* dY,
                   const float* W_hh, float* dc, float* dG, int64_t B, int64_t S, int64_t H,
                   hipStream_t st, const char* who) {
  const int64_t nbt = (B + 15) / 16, nbu = (H + 15) / 16;
  CNHIP_REQUIRE(nbt * nbu < ((int64_t)1 << 31), "%s: too many tiles", who);
  // FAST: full tiles, whole k-tiles, 16-byte aligned rows (dG is a scratch buffer)
  const bool fast = B % 16 == 0 && H % 16 == 0 && (4 * H) % Cfg::KT == 0 && (B * S) % 4 == 0 &&
                    aligned16(W_hh);
  const auto kern = fast ? &lstm_step_bwd_kernel<Cfg, true> : &lstm_step_bwd_kernel<Cfg, false>;
  for (int64_t t = S - 2; t >= 0; --t) {
    TimingRec* rec = timing_slot(2.0 * B * 4 * H * H);
    if (rec) (void)hipEventRecord(rec->start, st);
    hipLaunchKernelGGL(kern, dim3((unsigned)(nbt * nbu)), dim3(Cfg::NT), 0, st, gates, c, tanh_c, dY,
                       W_hh, dc, dG, B, S, H, t);
    CNHIP_TRY(check_launch(who));
    if (rec) (void)hipEventRecord(rec->stop, st);
  }
  return CNHIP_OK;
}

int check_rnn(int64_t B, int64_t S, int64_t I, int64_t H, const char* who) {
  CNHIP_REQUIRE(B > 0 && S > 0 && I > 0 && H > 0, "%s: bad shape B=%lld S=%lld I=%lld H=%lld", who,
                (long long)B, (long long)S, (long long)I, (long long)H);
  CNHIP_REQUIRE(B * H < ((int64_t)1 << 31), "%s: B*H too large", who);
  return CNHIP_OK;
}

struct Workspace {
  void* p = nullptr;
  hipStream_t st;
  explicit Workspace(hipStream_t s) : st(s) {}
  int alloc(size_t bytes, const char* who) { return scratch(st, kScratchLayer, bytes, &p, who); }
  ~Workspace() {
    // nothing to free: the stream's scratch slot is reused by later calls
  }
};

}  // namespace
}  // namespace cnhip

using cnhip::as_stream;

extern "C" {

int cnhip_lstm_forward(const float* X, const float* W_ih, const float* W_hh, const float* b,
                       float* Y, float* gates, float* c, float* tanh_c, int64_t B, int64_t S,
                       int64_t I, int64_t H, cnhip_stream_t stream) {
  const char* who = "cnhip_lstm_forward";
  CNHIP_TRY(cnhip::check_rnn(B, S, I, H, who));
  CNHIP_REQUIRE(X && W_ih && W_hh && b && Y && gates && c && tanh_c, "%s: NULL pointer", who);
  hipStream_t st = as_stream(stream);
  const int64_t G = 4 * H, BS = B * S;
  CNHIP_TRY(cnhip::gemm_f32(0, 0, BS, G, I, 1.f, X, BS, W_ih, I, 0.f, gates, BS, nullptr, 0, st, who));
  // t = 0: h_0 = 0, no recurrent term; then one fused GEMM + cell launch per step
  hipLaunchKernelGGL(cnhip::lstm_cell_fwd0_kernel, dim3(cnhip::cell_grid(B, H)), dim3(256), 0, st,
                     gates, b, c, tanh_c, Y, B, S, H);
  CNHIP_TRY(cnhip::check_launch(who));
  return cnhip::lstm_fwd_steps<cnhip::LstmFwdCfg>(gates, b, c, tanh_c, Y, W_hh, B, S, H, st, who);
}

int cnhip_lstm_backward(const float* X, const float* W_ih, const float* W_hh, const float* Y,
                        const float* gates, const float* c, const float* tanh_c, const float* dY,
                        float* gW_ih, float* gW_hh, float* gb, float* dX, int64_t B, int64_t S,
                        int64_t I, int64_t H, cnhip_stream_t stream) {
  const char* who = "cnhip_lstm_backward";
  CNHIP_TRY(cnhip::check_rnn(B, S, I, H, who));
  CNHIP_REQUIRE(X && W_ih && W_hh && Y && gates && c && tanh_c && dY && gW_ih && gW_hh && gb,
                "%s: NULL pointer", who);
  hipStream_t st = as_stream(stream);
  const int64_t G = 4 * H, BS = B * S;
  cnhip::Workspace ws(st);
  CNHIP_TRY(ws.alloc((size_t)(BS * G + B * H) * sizeof(float), who));
  float* dG = static_cast<float*>(ws.p);
  float* dc = dG + BS * G;
  // t = S-1: dh = dY only; then per step one fused launch of
  // dh_t = dY_t + dG_{t+1} W_hh^T (lstm.cpp:244) and the cell backward
  hipLaunchKernelGGL(cnhip::lstm_cell_bwd_last_kernel, dim3(cnhip::cell_grid(B, H)), dim3(256), 0,
                     st, gates, c, tanh_c, dY, dc, dG, B, S, H);
  CNHIP_TRY(cnhip::check_launch(who));
  CNHIP_TRY(cnhip::lstm_bwd_steps<cnhip::LstmBwdCfgDefault>(gates, c, tanh_c, dY, W_hh, dc, dG, B, S,
                                                            H, st, who));
  CNHIP_TRY(cnhip::gemm_f32(1, 0, I, G, BS, 1.f, X, BS, dG, BS, 0.f, gW_ih, I, nullptr, 0, st, who));
  CNHIP_TRY(cnhip::gemm_f32(1, 0, H, G, B * (S - 1), 1.f, Y, BS, dG + B, BS, 0.f, gW_hh, H, nullptr,
                            0, st, who));
  CNHIP_TRY(cnhip::column_sum(dG, gb, BS, G, 0, st, who));
  if (dX)
    CNHIP_TRY(cnhip::gemm_f32(0, 1, BS, I, G, 1.f, dG, BS, W_ih, I, 0.f, dX, BS, nullptr, 0, st, who));
  return CNHIP_OK;
}

int cnhip_gru_forward(const float* X, const float* W_ih, const float* W_hh, const float* b,
                      float* Y, float* gates, float* rh, int64_t B, int64_t S, int64_t I,
                      int64_t H, cnhip_stream_t stream) {
  const char* who = "cnhip_gru_forward";
  CNHIP_TRY(cnhip::check_rnn(B, S, I, H, who));
  CNHIP_REQUIRE(X && W_ih && W_hh && b && Y && gates && rh, "%s: NULL pointer", who);
  hipStream_t st = as_stream(stream);
  const int64_t G = 3 * H, BS = B * S;
  cnhip::Workspace ws(st);
  CNHIP_TRY(ws.alloc((size_t)(3 * B * H) * sizeof(float), who));
  float* hz = static_cast<float*>(ws.p);  // [B, 2H]
  float* proj = hz + 2 * B * H;           // [B, H]
  const float* W_hn = W_hh + H * 2 * H;
  CNHIP_TRY(cnhip::gemm_f32(0, 0, BS, G, I, 1.f, X, BS, W_ih, I, 0.f, gates, BS, nullptr, 0, st, who));
  for (int64_t t = 0; t < S; ++t) {
    if (t > 0)
      CNHIP_TRY(cnhip::gemm_f32(0, 0, B, 2 * H, H, 1.f, Y + B * (t - 1), BS, W_hh, H, 0.f, hz, B,
                                nullptr, 0, st, who));
    hipLaunchKernelGGL(cnhip::gru_zr_kernel, dim3(cnhip::cell_grid(B, H)), dim3(256), 0, st, gates,
                       hz, b, Y, rh, B, S, H, t);
    CNHIP_TRY(cnhip::check_launch(who));
    CNHIP_TRY(cnhip::gemm_f32(0, 0, B, H, H, 1.f, rh + B * t, BS, W_hn, H, 0.f, proj, B, nullptr, 0,
                              st, who));
    hipLaunchKernelGGL(cnhip::gru_n_kernel, dim3(cnhip::cell_grid(B, H)), dim3(256), 0, st, gates,
                       proj, b, Y, B, S, H, t);
    CNHIP_TRY(cnhip::check_launch(who));
  }
  return CNHIP_OK;
}

int cnhip_gru_backward(const float* X, const float* W_ih, const float* W_hh, const float* Y,
                       const float* gates, const float* rh, const float* dY, float* gW_ih,
                       float* gW_hh, float* gb, float* dX, int64_t B, int64_t S, int64_t I,
                       int64_t H, cnhip_stream_t stream) {
  const char* who = "cnhip_gru_backward";
  CNHIP_TRY(cnhip::check_rnn(B, S, I, H, who));
  CNHIP_REQUIRE(X && W_ih && W_hh && Y && gates && rh && dY && gW_ih && gW_hh && gb,
                "%s: NULL pointer", who);
  hipStream_t st = as_stream(stream);
  const int64_t G = 3 * H, BS = B * S;
  cnhip::Workspace ws(st);
  CNHIP_TRY(ws.alloc((size_t)(BS * G + 2 * B * H) * sizeof(float), who));
  float* dG = static_cast<float*>(ws.p);
  float* dh = dG + BS * G;
  float* drh = dh + B * H;
  const float* W_hn = W_hh + H * 2 * H;
  for (int64_t t = S - 1; t >= 0; --t) {
    hipLaunchKernelGGL(cnhip::gru_bwd_a_kernel, dim3(cnhip::cell_grid(B, H)), dim3(256), 0, st,
                       gates, Y, dY, dh, dG, B, S, H, t, t == S - 1 ? 1 : 0);
    CNHIP_TRY(cnhip::check_launch(who));
    // d_rh = dn_raw W_hn^T
    CNHIP_TRY(cnhip::gemm_f32(0, 1, B, H, H, 1.f, dG + B * t + BS * 2 * H, BS, W_hn, H, 0.f, drh, B,
                              nullptr, 0, st, who));
    hipLaunchKernelGGL(cnhip::gru_bwd_b_kernel, dim3(cnhip::cell_grid(B, H)), dim3(256), 0, st,
                       gates, Y, drh, dh, dG, B, S, H, t);
    CNHIP_TRY(cnhip::check_launch(who));
    // dh_next = dh_prev + dG_t[z,r] W_hh[:, 0:2H]^T
    if (t > 0)
      CNHIP_TRY(cnhip::gemm_f32(0, 1, B, H, 2 * H, 1.f, dG + B * t, BS, W_hh, H, 1.f, dh, B, nullptr,
                                0, st, who));
  }
  CNHIP_TRY(cnhip::gemm_f32(1, 0, I, G, BS, 1.f, X, BS, dG, BS, 0.f, gW_ih, I, nullptr, 0, st, who));
  CNHIP_TRY(cnhip::gemm_f32(1, 0, H, 2 * H, B * (S - 1), 1.f, Y, BS, dG + B, BS, 0.f, gW_hh, H,
                            nullptr, 0, st, who));
  CNHIP_TRY(cnhip::gemm_f32(1, 0, H, H, BS, 1.f, rh, BS, dG + BS * 2 * H, BS, 0.f, gW_hh + H * 2 * H,
                            H, nullptr, 0, st, who));
  CNHIP_TRY(cnhip::column_sum(dG, gb, BS, G, 0, st, who));
  if (dX)
    CNHIP_TRY(cnhip::gemm_f32(0, 1, BS, I, G, 1.f, dG, BS, W_ih, I, 0.f, dX, BS, nullptr, 0, st, who));
  return CNHIP_OK;
}

int cnhip_seq_select(const float* Y, float* out, int64_t B, int64_t S, int64_t D, int64_t t,
                     cnhip_stream_t stream) {
  const char* who = "cnhip_seq_select";
  CNHIP_REQUIRE(B > 0 && S > 0 && D > 0 && t >= 0 && t < S, "%s: bad shape or step", who);
  CNHIP_REQUIRE(Y && out, "%s: NULL pointer", who);
  cnhip::HbmTimer timer("seq_select_kernel", 8.0 * (double)B * (double)D, as_stream(stream));
  hipLaunchKernelGGL(cnhip::seq_select_kernel, dim3((unsigned)((B * D + 255) / 256)), dim3(256), 0,
                     as_stream(stream), Y, out, B, S, D, t);
  return cnhip::check_launch(who);
}

int cnhip_seq_scatter(const float* in, float* Y, int64_t B, int64_t S, int64_t D, int64_t t,
                      cnhip_stream_t stream) {
  const char* who = "cnhip_seq_scatter";
  CNHIP_REQUIRE(B > 0 && S > 0 && D > 0 && t >= 0 && t < S, "%s: bad shape or step", who);
  CNHIP_REQUIRE(Y && in, "%s: NULL pointer", who);
  // the step's rows read; the whole sequence gradient written (zeros elsewhere)
  cnhip::HbmTimer timer("seq_scatter_kernel", 4.0 * (double)B * (double)D * (double)(S + 1),
                        as_stream(stream));
  hipLaunchKernelGGL(cnhip::seq_scatter_kernel, dim3(cnhip::elementwise_grid(B * S * D, 256)),
                     dim3(256), 0, as_stream(stream), in, Y, B, S, D, t);
  return cnhip::check_launch(who);
}

int cnhip_rnn_forward(const float* X, const float* W_ih, const float* W_hh, const float* b, float* Y,
                      int64_t B, int64_t S, int64_t I, int64_t H, cnhip_stream_t stream) {
  const char* who = "cnhip_rnn_forward";
  CNHIP_REQUIRE(B > 0 && S > 0 && I > 0 && H > 0, "%s: bad shape B=%lld S=%lld I=%lld H=%lld", who,
                (long long)B, (long long)S, (long long)I, (long long)H);
  CNHIP_REQUIRE(X && W_ih && W_hh && b && Y, "%s: NULL pointer", who);
  hipStream_t st = as_stream(stream);
  const int64_t BS = B * S;
  // x_t W_ih for every step at once (rnn.cpp:73-74), then the recurrence:
  // step t's rows of Y = tanh(h_{t-1} W_hh + Y_t + b), the GEMM adding the
  // x-projection (beta = 1) and the bias and applying tanh in its epilogue
  CNHIP_TRY(cnhip::gemm_f32(0, 0, BS, H, I, 1.f, X, BS, W_ih, I, 0.f, Y, BS, nullptr, 0, st, who));
  hipLaunchKernelGGL(cnhip::rnn_step0_kernel, dim3(cnhip::cell_grid(B, H)), dim3(256), 0, st, Y, b, B, BS, H);
  CNHIP_TRY(cnhip::check_launch(who));
  for (int64_t t = 1; t < S; ++t)
    CNHIP_TRY(cnhip::gemm_f32_core(0, 0, B, H, H, 1.f, Y + B * (t - 1), BS, 0, W_hh, H, 0, 1.f, Y + B * t, BS,
                                   0, 1, b, cnhip::EPI_TANH, nullptr, nullptr, 0, st, who));
  return CNHIP_OK;
}

int cnhip_rnn_backward(const float* X, const float* W_ih, const float* W_hh, const float* Y, const float* dY,
                       float* gW_ih, float* gW_hh, float* gb, float* dX, int64_t B, int64_t S, int64_t I,
                       int64_t H, cnhip_stream_t stream) {
  const char* who = "cnhip_rnn_backward";
  CNHIP_REQUIRE(B > 0 && S > 0 && I > 0 && H > 0, "%s: bad shape", who);
  CNHIP_REQUIRE(X && W_ih && W_hh && Y && dY && gW_ih && gW_hh && gb, "%s: NULL pointer", who);
  hipStream_t st = as_stream(stream);
  const int64_t BS = B * S;
  cnhip::Workspace ws(st);
  CNHIP_TRY(ws.alloc((size_t)(BS * H + B * H) * sizeof(float), who));
  float* dT = static_cast<float*>(ws.p);  // dtanh of every step, [B*S, H]
  float* dh = dT + BS * H;                // dh_next = dtanh_{t+1} W_hh^T, [B, H]
  for (int64_t t = S - 1; t >= 0; --t) {
    hipLaunchKernelGGL(cnhip::rnn_bwd_cell_kernel, dim3(cnhip::cell_grid(B, H)), dim3(256), 0, st, dY, Y,
                       t == S - 1 ? nullptr : dh, dT, B, BS, H, t);
    CNHIP_TRY(cnhip::check_launch(who));
    if (t > 0)
      CNHIP_TRY(cnhip::gemm_f32(0, 1, B, H, H, 1.f, dT + B * t, BS, W_hh, H, 0.f, dh, B, nullptr, 0, st, who));
  }
  // weight grads over all B*S rows (rnn.cpp:136-142): gW_ih = X^T dT,
  // gW_hh = [h_0 .. h_{S-2}]^T dT[steps 1..S-1] (h_{-1} = 0 adds nothing),
  // gb = colsum dT; dX = dT W_ih^T (rnn.cpp:145-149)
  CNHIP_TRY(cnhip::gemm_f32(1, 0, I, H, BS, 1.f, X, BS, dT, BS, 0.f, gW_ih, I, nullptr, 0, st, who));
  if (S > 1)
    CNHIP_TRY(cnhip::gemm_f32(1, 0, H, H, B * (S - 1), 1.f, Y, BS, dT + B, BS, 0.f, gW_hh, H, nullptr, 0, st,
                              who));
  else
    CNHIP_TRY(cnhip::fill_bytes(gW_hh, 0, (size_t)(H * H) * sizeof(float), st, who));
  CNHIP_TRY(cnhip::column_sum(dT, gb, BS, H, 0, st, who));
  if (dX) CNHIP_TRY(cnhip::gemm_f32(0, 1, BS, I, H, 1.f, dT, BS, W_ih, I, 0.f, dX, BS, nullptr, 0, st, who));
  return CNHIP_OK;
}

}  // extern "C"
