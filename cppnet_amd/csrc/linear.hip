// Linear layer entry points and the bias-gradient column reduction.
//
// ref: Linear::forward_gpu / backward_gpu, src/CppNet/layers/linear.cpp:456-539
// and the cpu-eigen semantics they must match, linear.cpp:218-234, 335-358:
//   Y  = X W + b
//   dW += X^T dY      db += sum_batch dY      dX = dY W^T
#include <hip/hip_runtime.h>

#include "common.hpp"

namespace cnhip {

int linear_wgrad_small(const float* X, const float* dY, float* dW, float* db, int64_t batch,
                       int64_t in_features, int64_t out_features, int accumulate, hipStream_t st,
                       const char* who, bool* done);
int gemm_f32(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha,
             const float* A, int64_t lda, const float* B, int64_t ldb, float beta, float* C,
             int64_t ldc, const float* bias, int epilogue, hipStream_t st, const char* who);
int gemm_f32_act(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, const float* A,
                 int64_t lda, const float* B, int64_t ldb, float* C, int64_t ldc, const float* bias,
                 int epilogue, const float* aux_in, float* aux_out, int64_t ld_aux, hipStream_t st,
                 const char* who);
// fused-activation epilogue codes of gemm_f32_act
constexpr int EPI_GELU = 2, EPI_DRELU = 3, EPI_DGELU = 4, EPI_ADD = 5;

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// One wavefront per column of a ColMajor [rows, cols] matrix; a column is
// contiguous, so each lane streams float4s and the wave reduces with DPP/
// shuffles.  The summation order is fixed, so results are deterministic.
__global__ void __launch_bounds__(256) column_sum_kernel(const float* __restrict__ in,
                                                         float* __restrict__ out, int64_t rows,
                                                         int64_t cols, int accumulate, int vec) {
  const int lane = threadIdx.x & 63;
  const int64_t col = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (col >= cols) return;
  const float* p = in + rows * col;
  float s = 0.f;
  if (vec) {
    // four float4 loads in flight per lane, four running sums added in order
    const int64_t n4 = rows >> 2;
    const f32x4* p4 = reinterpret_cast<const f32x4*>(p);
    f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = a0, a2 = a0, a3 = a0;
    int64_t i = lane;
    for (; i + 192 < n4; i += 256) {
      a0 += p4[i];
      a1 += p4[i + 64];
      a2 += p4[i + 128];
      a3 += p4[i + 192];
    }
    for (; i < n4; i += 64) a0 += p4[i];
    const f32x4 t = (a0 + a1) + (a2 + a3);
    s = (t[0] + t[1]) + (t[2] + t[3]);
  } else {
    for (int64_t i = lane; i < rows; i += 64) s += p[i];
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  if (lane == 0) out[col] = accumulate ? out[col] + s : s;
}

}  // namespace

int column_sum(const float* in, float* out, int64_t rows, int64_t cols, int accumulate,
               hipStream_t st, const char* who) {
  CNHIP_REQUIRE(rows >= 0 && cols >= 0, "%s: negative size", who);
  if (cols == 0) return CNHIP_OK;
  CNHIP_REQUIRE(out != nullptr, "%s: out is NULL", who);
  CNHIP_REQUIRE(rows == 0 || in != nullptr, "%s: in is NULL", who);
  const int vec = (rows % 4 == 0) && aligned16(in);
  HbmTimer timer("column_sum_kernel", 4.0 * (double)rows * (double)cols + (accumulate ? 8.0 : 4.0) * (double)cols,
                 st);
  hipLaunchKernelGGL(column_sum_kernel, dim3((unsigned)((cols + 3) / 4)), dim3(256), 0, st, in, out,
                     rows, cols, accumulate, vec);
  return check_launch(who);
}

}  // namespace cnhip

extern "C" {

int cnhip_column_sum(const float* in, float* out, int64_t rows, int64_t cols, int accumulate,
                     cnhip_stream_t stream) {
  return cnhip::column_sum(in, out, rows, cols, accumulate, cnhip::as_stream(stream),
                           "cnhip_column_sum");
}

int cnhip_linear_forward(const float* X, const float* W, const float* b, float* Y, int64_t batch,
                         int64_t in_features, int64_t out_features, cnhip_stream_t stream) {
  CNHIP_REQUIRE(batch >= 0 && in_features > 0 && out_features > 0,
                "cnhip_linear_forward: bad shape batch=%lld in=%lld out=%lld", (long long)batch,
                (long long)in_features, (long long)out_features);
  // Y[B,O] = X[B,I] * W[I,O]  (+ b)
  return cnhip::gemm_f32(0, 0, batch, out_features, in_features, 1.f, X, batch, W, in_features,
                         0.f, Y, batch, b, CNHIP_EPI_NONE, cnhip::as_stream(stream),
                         "cnhip_linear_forward");
}

int cnhip_linear_backward(const float* X, const float* W, const float* dY, float* grad_W,
                          float* grad_b, float* dX, int64_t batch, int64_t in_features,
                          int64_t out_features, int trainable, int accumulate,
                          cnhip_stream_t stream) {
  const char* who = "cnhip_linear_backward";
  CNHIP_REQUIRE(batch >= 0 && in_features > 0 && out_features > 0,
                "%s: bad shape batch=%lld in=%lld out=%lld", who, (long long)batch,
                (long long)in_features, (long long)out_features);
  hipStream_t st = cnhip::as_stream(stream);
  const float beta = accumulate ? 1.f : 0.f;
  if (trainable) {
    CNHIP_REQUIRE(grad_W != nullptr, "%s: trainable layer needs grad_W", who);
    // dW[I,O] (+)= X^T[I,B] * dY[B,O]; db (+)= the column sums of dY (one
    // launch for both when the GEMM is small enough for the SIMT kernels)
    bool fused = false;
    CNHIP_TRY(cnhip::linear_wgrad_small(X, dY, grad_W, grad_b, batch, in_features, out_features, accumulate,
                                        st, who, &fused));
    if (!fused) {
      CNHIP_TRY(cnhip::gemm_f32(1, 0, in_features, out_features, batch, 1.f, X, batch, dY, batch,
                                beta, grad_W, in_features, nullptr, CNHIP_EPI_NONE, st, who));
      if (grad_b) CNHIP_TRY(cnhip::column_sum(dY, grad_b, batch, out_features, accumulate, st, who));
    }
  }
  if (dX) {
    // dX[B,I] = dY[B,O] * W^T[O,I]
    CNHIP_TRY(cnhip::gemm_f32(0, 1, batch, in_features, out_features, 1.f, dY, batch, W,
                              in_features, 0.f, dX, batch, nullptr, CNHIP_EPI_NONE, st, who));
  }
  return CNHIP_OK;
}

int cnhip_linear_forward_act(const float* X, const float* W, const float* b, float* Y, float* Z,
                             int64_t batch, int64_t in_features, int64_t out_features, int act,
                             cnhip_stream_t stream) {
  const char* who = "cnhip_linear_forward_act";
  CNHIP_REQUIRE(batch >= 0 && in_features > 0 && out_features > 0, "%s: bad shape", who);
  CNHIP_REQUIRE(act >= CNHIP_ACT_NONE && act <= CNHIP_ACT_RESIDUAL, "%s: bad activation %d", who, act);
  CNHIP_REQUIRE(act != CNHIP_ACT_GELU || Z, "%s: GELU needs Z for the pre-activation", who);
  CNHIP_REQUIRE(act != CNHIP_ACT_RESIDUAL || Z, "%s: the residual add needs Z (the residual input)", who);
  const int epi = act == CNHIP_ACT_RELU       ? CNHIP_EPI_RELU
                  : act == CNHIP_ACT_GELU     ? cnhip::EPI_GELU
                  : act == CNHIP_ACT_RESIDUAL ? cnhip::EPI_ADD
                                              : CNHIP_EPI_NONE;
  return cnhip::gemm_f32_act(0, 0, batch, out_features, in_features, X, batch, W, in_features, Y,
                             batch, b, epi, act == CNHIP_ACT_RESIDUAL ? Z : nullptr,
                             act == CNHIP_ACT_GELU ? Z : nullptr, batch, cnhip::as_stream(stream), who);
}

int cnhip_linear_backward_act(const float* X, const float* W, const float* dY, float* grad_W,
                              float* grad_b, float* dX, const float* act_aux, int64_t batch,
                              int64_t in_features, int64_t out_features, int trainable,
                              int accumulate, int act, cnhip_stream_t stream) {
  const char* who = "cnhip_linear_backward_act";
  CNHIP_REQUIRE(act >= CNHIP_ACT_NONE && act <= CNHIP_ACT_RESIDUAL, "%s: bad activation %d", who, act);
  CNHIP_REQUIRE(act == CNHIP_ACT_NONE || (dX && act_aux), "%s: activation %d needs dX and act_aux",
                who, act);
  CNHIP_TRY(cnhip_linear_backward(X, W, dY, grad_W, grad_b, act == CNHIP_ACT_NONE ? dX : nullptr,
                                  batch, in_features, out_features, trainable, accumulate, stream));
  if (act == CNHIP_ACT_NONE || batch == 0) return CNHIP_OK;
  // dX[B,I] = (dY W^T) * act'(act_aux), the activation's backward in the
  // epilogue; for the residual, dX = dY W^T + act_aux (the skip branch's gradient)
  const int epi = act == CNHIP_ACT_RELU   ? cnhip::EPI_DRELU
                  : act == CNHIP_ACT_GELU ? cnhip::EPI_DGELU
                                          : cnhip::EPI_ADD;
  return cnhip::gemm_f32_act(0, 1, batch, in_features, out_features, dY, batch, W, in_features, dX,
                             batch, nullptr, epi, act_aux, nullptr, batch, cnhip::as_stream(stream),
                             who);
}

}  // extern "C"
