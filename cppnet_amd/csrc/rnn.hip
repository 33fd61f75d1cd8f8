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
//   forward : G = X W_ih (all steps)       then per step G_t += h_{t-1} W_hh
//   backward: per step only the cell kernel and dh_{t-1} = dG_t W_hh^T;
//             afterwards dW_ih = X^T dG, dW_hh = Y_{t-1}^T dG, db = colsum dG,
//             dX = dG W_ih^T, each a single GEMM over all B*S rows.
// The cell kernels fuse every elementwise gate computation of a step into one
// pass (one thread per (n, d); n fastest for coalescing) and evaluate the
// reference expressions in the reference's operation order.
#include <hip/hip_runtime.h>

#include <cmath>

#include "common.hpp"

namespace cnhip {

int gemm_f32(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha,
             const float* A, int64_t lda, const float* B, int64_t ldb, float beta, float* C,
             int64_t ldc, const float* bias, int epilogue, hipStream_t st, const char* who);
int column_sum(const float* in, float* out, int64_t rows, int64_t cols, int accumulate,
               hipStream_t st, const char* who);
int gemm_f32_partials(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K,
                      const float* A, int64_t lda, const float* B, int64_t ldb, float* partial,
                      int max_splits, int* splits_out, hipStream_t st, const char* who);

namespace {

__device__ __forceinline__ float sigm(float x) { return 1.0f / (1.0f + expf(-x)); }

// Sum of nsplit split-K partials p[z*stride + i], z ascending (0 when nsplit
// is 0): the recurrent GEMM's output, reduced inside the cell kernel that
// consumes it instead of by a separate pass.
__device__ __forceinline__ float partial_sum(const float* __restrict__ p, int nsplit,
                                             int64_t stride, int64_t i) {
  float s = 0.0f;
#pragma unroll 4
  for (int z = 0; z < nsplit; ++z) s += p[z * stride + i];
  return s;
}

// ---------------------------------------------------------------- LSTM cell
// gates rows of step t hold x W_ih; the recurrent part h_{t-1} W_hh arrives as
// nsplit split-K partials hw[z][n + B*j] (j < 4H).  The pre-activations
// (x W_ih + h W_hh) are overwritten with the activations i, f, g, o
// (lstm.cpp:115-134).
__global__ void __launch_bounds__(256) lstm_cell_fwd_kernel(float* __restrict__ gates,
                                                            const float* __restrict__ bias,
                                                            float* __restrict__ c,
                                                            float* __restrict__ tanh_c,
                                                            float* __restrict__ Y,
                                                            const float* __restrict__ hw,
                                                            int nsplit, int64_t B, int64_t S,
                                                            int64_t H, int64_t t) {
  const int64_t BS = B * S, BG = B * 4 * H;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= B * H) return;
  const int64_t n = e % B, d = e / B, row = n + B * t;
  float* g = gates + row;
  auto pre = [&](int64_t j) {
    const float x = g[BS * j];
    return nsplit ? partial_sum(hw, nsplit, BG, n + B * j) + x : x;
  };
  const float ig = sigm(pre(d) + bias[d]);
  const float fg = sigm(pre(d + H) + bias[d + H]);
  const float gg = tanhf(pre(d + 2 * H) + bias[d + 2 * H]);
  const float og = sigm(pre(d + 3 * H) + bias[d + 3 * H]);
  const float cprev = t > 0 ? c[row - B + BS * d] : 0.0f;
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

// lstm.cpp:184-219, 247-249.  dh_in: the nsplit split-K partials of
// dG_{t+1} W_hh^T, [z][B, H]; dc: [B, H] (dense, ld B); both ignored when first.
__global__ void __launch_bounds__(256) lstm_cell_bwd_kernel(
    const float* __restrict__ gates, const float* __restrict__ c, const float* __restrict__ tanh_c,
    const float* __restrict__ dY, const float* __restrict__ dh_in, int nsplit,
    float* __restrict__ dc_buf, float* __restrict__ dG, int64_t B, int64_t S, int64_t H, int64_t t,
    int first) {
  const int64_t BS = B * S;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= B * H) return;
  const int64_t n = e % B, d = e / B, row = n + B * t;
  const float ig = gates[row + BS * d], fg = gates[row + BS * (d + H)];
  const float gg = gates[row + BS * (d + 2 * H)], og = gates[row + BS * (d + 3 * H)];
  const float tc = tanh_c[row + BS * d];
  const float dh = dY[row + BS * d] + (first ? 0.0f : partial_sum(dh_in, nsplit, B * H, e));
  const float dc = dh * og * (1.0f - tc * tc) + (first ? 0.0f : dc_buf[e]);
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
  constexpr int kMaxSplits = 8;
  cnhip::Workspace ws(st);
  CNHIP_TRY(ws.alloc((size_t)kMaxSplits * B * G * sizeof(float), who));
  float* hw = static_cast<float*>(ws.p);
  CNHIP_TRY(cnhip::gemm_f32(0, 0, BS, G, I, 1.f, X, BS, W_ih, I, 0.f, gates, BS, nullptr, 0, st, who));
  for (int64_t t = 0; t < S; ++t) {
    int ns = 0;  // h_0 = 0: no recurrent term at t = 0
    if (t > 0)
      CNHIP_TRY(cnhip::gemm_f32_partials(0, 0, B, G, H, Y + B * (t - 1), BS, W_hh, H, hw, kMaxSplits,
                                         &ns, st, who));
    hipLaunchKernelGGL(cnhip::lstm_cell_fwd_kernel, dim3(cnhip::cell_grid(B, H)), dim3(256), 0, st,
                       gates, b, c, tanh_c, Y, hw, ns, B, S, H, t);
    CNHIP_TRY(cnhip::check_launch(who));
  }
  return CNHIP_OK;
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
  constexpr int kMaxSplits = 16;
  cnhip::Workspace ws(st);
  CNHIP_TRY(ws.alloc((size_t)(BS * G + (kMaxSplits + 1) * B * H) * sizeof(float), who));
  float* dG = static_cast<float*>(ws.p);
  float* dc = dG + BS * G;
  float* dh = dc + B * H;  // kMaxSplits partials of dG_t W_hh^T
  int ns = 0;
  for (int64_t t = S - 1; t >= 0; --t) {
    hipLaunchKernelGGL(cnhip::lstm_cell_bwd_kernel, dim3(cnhip::cell_grid(B, H)), dim3(256), 0, st,
                       gates, c, tanh_c, dY, dh, ns, dc, dG, B, S, H, t, t == S - 1 ? 1 : 0);
    CNHIP_TRY(cnhip::check_launch(who));
    if (t > 0)  // dh_next = dG_t W_hh^T (lstm.cpp:244), summed by the next cell kernel
      CNHIP_TRY(cnhip::gemm_f32_partials(0, 1, B, H, G, dG + B * t, BS, W_hh, H, dh, kMaxSplits, &ns,
                                         st, who));
  }
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
  hipLaunchKernelGGL(cnhip::seq_select_kernel, dim3((unsigned)((B * D + 255) / 256)), dim3(256), 0,
                     as_stream(stream), Y, out, B, S, D, t);
  return cnhip::check_launch(who);
}

int cnhip_seq_scatter(const float* in, float* Y, int64_t B, int64_t S, int64_t D, int64_t t,
                      cnhip_stream_t stream) {
  const char* who = "cnhip_seq_scatter";
  CNHIP_REQUIRE(B > 0 && S > 0 && D > 0 && t >= 0 && t < S, "%s: bad shape or step", who);
  CNHIP_REQUIRE(Y && in, "%s: NULL pointer", who);
  hipLaunchKernelGGL(cnhip::seq_scatter_kernel, dim3(cnhip::elementwise_grid(B * S * D, 256)),
                     dim3(256), 0, as_stream(stream), in, Y, B, S, D, t);
  return cnhip::check_launch(who);
}

}  // extern "C"
