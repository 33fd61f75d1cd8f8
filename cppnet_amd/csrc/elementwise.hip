// Bandwidth-bound kernels: activation forward/backward and the loss
// functions of the hot path.  Each activation kernel streams float4s
// through a grid-stride loop sized to fill the 256 CUs.  Loss values are
// reduced in a fixed order (deterministic, no atomics): BCE and MSE in one
// block, softmax-CE per row block and then over the block partials.
//
// Arithmetic follows the cpu-eigen branches operation by operation:
//   ReLU     relu.cpp:97-225          Sigmoid   sigmoid.cpp:97-231
//   Tanh     tanh.cpp:136-219         BCE       binary_cross_entropy.cpp:143-225
//   MSE      mse.cpp:102-161          SoftmaxCE softmax_cross_entropy.cpp:118-195
#include <hip/hip_runtime.h>

#include "act_math.hpp"
#include "common.hpp"

namespace cnhip {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

struct ReluFwd {
  static constexpr const char* kKernel = "unary_kernel<ReluFwd>";
  __device__ float operator()(float x) const { return relu_f(x); }
};
struct SigmoidFwd {
  static constexpr const char* kKernel = "unary_kernel<SigmoidFwd>";
  __device__ float operator()(float x) const {
    const float c = fmaxf(-500.f, fminf(500.f, x));
    return 1.f / (1.f + expf(-c));
  }
};
struct TanhFwd {
  static constexpr const char* kKernel = "unary_kernel<TanhFwd>";
  __device__ float operator()(float x) const { return tanhf(x); }
};
// grad_output * mask, mask = 1 where the cached output is > 0 (relu.cpp:177-181)
struct ReluBwd {
  static constexpr const char* kKernel = "binary_kernel<ReluBwd>";
  __device__ float operator()(float y, float dy) const { return dy * relu_mask(y); }
};
// grad_output * (s * (1 - s))  (sigmoid.cpp:192-194)
struct SigmoidBwd {
  static constexpr const char* kKernel = "binary_kernel<SigmoidBwd>";
  __device__ float operator()(float y, float dy) const { return dy * (y * (1.f - y)); }
};
// grad_output * (1 - t*t)  (tanh.cpp:153-154)
struct TanhBwd {
  static constexpr const char* kKernel = "binary_kernel<TanhBwd>";
  __device__ float operator()(float y, float dy) const { return dy * (1.f - y * y); }
};

template <class Op>
__global__ void __launch_bounds__(256) unary_kernel(const float* __restrict__ x,
                                                    float* __restrict__ y, int64_t n, int vec) {
  Op op;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (vec) {
    const int64_t n4 = n >> 2;
    for (int64_t i = t0; i < n4; i += stride) {
      f32x4 v = reinterpret_cast<const f32x4*>(x)[i];
      f32x4 r;
      r[0] = op(v[0]); r[1] = op(v[1]); r[2] = op(v[2]); r[3] = op(v[3]);
      reinterpret_cast<f32x4*>(y)[i] = r;
    }
  } else {
    for (int64_t i = t0; i < n; i += stride) y[i] = op(x[i]);
  }
}

template <class Op>
__global__ void __launch_bounds__(256) binary_kernel(const float* __restrict__ y,
                                                     const float* __restrict__ dy,
                                                     float* __restrict__ dx, int64_t n, int vec) {
  Op op;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (vec) {
    const int64_t n4 = n >> 2;
    for (int64_t i = t0; i < n4; i += stride) {
      f32x4 a = reinterpret_cast<const f32x4*>(y)[i];
      f32x4 b = reinterpret_cast<const f32x4*>(dy)[i];
      f32x4 r;
      r[0] = op(a[0], b[0]); r[1] = op(a[1], b[1]); r[2] = op(a[2], b[2]); r[3] = op(a[3], b[3]);
      reinterpret_cast<f32x4*>(dx)[i] = r;
    }
  } else {
    for (int64_t i = t0; i < n; i += stride) dx[i] = op(y[i], dy[i]);
  }
}

template <class Op>
int launch_unary(const float* x, float* y, int64_t n, hipStream_t st, const char* who) {
  CNHIP_REQUIRE(n >= 0, "%s: negative size", who);
  if (n == 0) return CNHIP_OK;
  CNHIP_REQUIRE(x && y, "%s: NULL pointer", who);
  const int vec = (n % 4 == 0) && aligned16(x) && aligned16(y);
  const int64_t items = vec ? n / 4 : n;
  HbmTimer timer(Op::kKernel, 8.0 * (double)n, st);
  hipLaunchKernelGGL(unary_kernel<Op>, dim3(elementwise_grid(items, 256)), dim3(256), 0, st, x, y,
                     n, vec);
  return check_launch(who);
}

template <class Op>
int launch_binary(const float* y, const float* dy, float* dx, int64_t n, hipStream_t st,
                  const char* who) {
  CNHIP_REQUIRE(n >= 0, "%s: negative size", who);
  if (n == 0) return CNHIP_OK;
  CNHIP_REQUIRE(y && dy && dx, "%s: NULL pointer", who);
  const int vec = (n % 4 == 0) && aligned16(y) && aligned16(dy) && aligned16(dx);
  const int64_t items = vec ? n / 4 : n;
  HbmTimer timer(Op::kKernel, 12.0 * (double)n, st);
  hipLaunchKernelGGL(binary_kernel<Op>, dim3(elementwise_grid(items, 256)), dim3(256), 0, st, y,
                     dy, dx, n, vec);
  return check_launch(who);
}

// ---- block reduction (1024 threads, fixed order) -------------------------
constexpr int RB = 1024;

__device__ float block_sum(float v, float* smem) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  if (lane == 0) smem[wave] = v;
  __syncthreads();
  float r = 0.f;
  if (threadIdx.x == 0)
    for (int w = 0; w < RB / 64; ++w) r += smem[w];
  return r;  // valid on thread 0
}

__device__ __forceinline__ float bce_clip(float p) { return fmaxf(1e-7f, fminf(p, 1.0f - 1e-7f)); }

__global__ void __launch_bounds__(RB) bce_forward_kernel(const float* __restrict__ p,
                                                         const float* __restrict__ t,
                                                         float* __restrict__ loss, int64_t n,
                                                         int reduction) {
  __shared__ float smem[RB / 64];
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += RB) {
    const float pc = bce_clip(p[i]);
    const float tv = t[i];
    s += -(tv * logf(pc) + (1.0f - tv) * logf(1.0f - pc));
  }
  const float tot = block_sum(s, smem);
  if (threadIdx.x == 0) *loss = (reduction == CNHIP_REDUCE_SUM) ? tot : tot / (float)n;
}

// grad = (p - t) / (p (1 - p)) with the denominator in double, then / n in
// float, as binary_cross_entropy.cpp:209-218 computes it.
__global__ void __launch_bounds__(256) bce_backward_kernel(const float* __restrict__ p,
                                                           const float* __restrict__ t,
                                                           float* __restrict__ g, int64_t n,
                                                           int reduction) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float pc = bce_clip(p[i]);
    const float diff = pc - t[i];
    float gv = (float)((double)diff / ((double)pc * (1.0 - (double)pc)));
    if (reduction == CNHIP_REDUCE_MEAN) gv /= (float)n;
    g[i] = gv;
  }
}

// Sigmoid output layer + BinaryCrossEntropy, forward and backward, in one
// single-block launch for small outputs: per element the four separate
// kernels' arithmetic (SigmoidFwd, the BCE term, the BCE gradient, SigmoidBwd)
// and the loss's per-thread partial sums over the same elements as
// bce_forward_kernel, so every output is bit-identical to the four launches.
__global__ void __launch_bounds__(RB) sigmoid_bce_head_kernel(const float* __restrict__ z,
                                                              const float* __restrict__ t,
                                                              float* __restrict__ p,
                                                              float* __restrict__ loss,
                                                              float* __restrict__ dz, int64_t n,
                                                              int loss_reduction, int grad_reduction) {
  __shared__ float smem[RB / 64];
  const SigmoidFwd sig;
  const SigmoidBwd dsig;
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += RB) {
    const float pv = sig(z[i]);
    p[i] = pv;
    const float pc = bce_clip(pv);
    const float tv = t[i];
    s += -(tv * logf(pc) + (1.0f - tv) * logf(1.0f - pc));
    const float diff = pc - tv;
    float gv = (float)((double)diff / ((double)pc * (1.0 - (double)pc)));
    if (grad_reduction == CNHIP_REDUCE_MEAN) gv /= (float)n;
    dz[i] = dsig(pv, gv);
  }
  const float tot = block_sum(s, smem);
  if (threadIdx.x == 0) *loss = (loss_reduction == CNHIP_REDUCE_SUM) ? tot : tot / (float)n;
}

__global__ void __launch_bounds__(RB) mse_forward_kernel(const float* __restrict__ p,
                                                         const float* __restrict__ t,
                                                         float* __restrict__ loss, int64_t n,
                                                         int reduction) {
  __shared__ float smem[RB / 64];
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += RB) {
    const float d = p[i] - t[i];
    s += d * d;
  }
  const float tot = block_sum(s, smem);
  if (threadIdx.x == 0) *loss = (reduction == CNHIP_REDUCE_MEAN) ? tot / (float)n : tot;
}

// MSE forward and backward in one single-block launch for small outputs:
// the loss's per-thread partial sums over the same elements as
// mse_forward_kernel and each gradient element as mse_backward_kernel forms
// it, so loss and gradient are bit-identical to the two launches.
__global__ void __launch_bounds__(RB) mse_head_kernel(const float* __restrict__ p, const float* __restrict__ t,
                                                      float* __restrict__ loss, float* __restrict__ g, int64_t n,
                                                      int loss_reduction, float grad_scale) {
  __shared__ float smem[RB / 64];
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += RB) {
    const float d = p[i] - t[i];
    s += d * d;
    g[i] = grad_scale * d;
  }
  const float tot = block_sum(s, smem);
  if (threadIdx.x == 0) *loss = (loss_reduction == CNHIP_REDUCE_MEAN) ? tot / (float)n : tot;
}

__global__ void __launch_bounds__(256) mse_backward_kernel(const float* __restrict__ p,
                                                           const float* __restrict__ t,
                                                           float* __restrict__ g, int64_t n,
                                                           float scale) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    g[i] = scale * (p[i] - t[i]);
}

// Softmax-CE over ColMajor [B, C]: row b lives at b + B*c, so consecutive
// threads take consecutive rows and every class loop reads coalesced.  Each
// block writes the sum of its rows' losses to partial[blockIdx.x]; a second
// single-block kernel adds the partials in block order (deterministic).
constexpr int SCE_BLOCK = 256;

__global__ void __launch_bounds__(SCE_BLOCK) softmax_ce_rows_kernel(
    const float* __restrict__ z, const float* __restrict__ t, float* __restrict__ sm,
    float* __restrict__ partial, int64_t B, int64_t C) {
  __shared__ float smem[SCE_BLOCK / 64];
  float row = 0.f;
  const int64_t b = (int64_t)blockIdx.x * SCE_BLOCK + threadIdx.x;
  if (b < B) {
    float mx = z[b];
    for (int64_t c = 1; c < C; ++c) mx = fmaxf(mx, z[b + B * c]);
    float se = 0.f;
    for (int64_t c = 0; c < C; ++c) {
      const float e = expf(z[b + B * c] - mx);
      sm[b + B * c] = e;
      se += e;
    }
    const float ls = logf(se + 1e-12f);
    for (int64_t c = 0; c < C; ++c) {
      sm[b + B * c] = sm[b + B * c] / se;
      row -= t[b + B * c] * ((z[b + B * c] - mx) - ls);
    }
  }
  // fixed-order block sum
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) row += __shfl_xor(row, off, 64);
  if (lane == 0) smem[wave] = row;
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = 0.f;
    for (int w = 0; w < SCE_BLOCK / 64; ++w) s += smem[w];
    partial[blockIdx.x] = s;
  }
}

// softmax_ce_rows_kernel + the backward for B <= SCE_BLOCK rows in one block:
// the same per-row arithmetic and fixed-order block sum; the loss is that sum
// over the divisor, which is what partial_sum_kernel makes of a single
// partial (it adds only zeros to it).  Gradient as softmax_ce_backward_kernel.
// REG > 0: a row of at most REG classes is loaded once into registers (the
// same values, so the same results, without re-reading memory per pass).
template <int REG>
__global__ void __launch_bounds__(SCE_BLOCK) softmax_ce_head_kernel(
    const float* __restrict__ z, const float* __restrict__ t, float* __restrict__ sm,
    float* __restrict__ loss, float* __restrict__ g, int64_t B, int64_t C, float divisor, int mean,
    float inv_batch) {
  __shared__ float smem[SCE_BLOCK / 64];
  float row = 0.f;
  const int64_t b = threadIdx.x;
  if (REG > 0 && b < B) {
    float zr[REG > 0 ? REG : 1], tr[REG > 0 ? REG : 1];
#pragma unroll
    for (int c = 0; c < REG; ++c) {
      zr[c] = c < C ? z[b + B * c] : 0.f;
      tr[c] = c < C ? t[b + B * c] : 0.f;
    }
    float mx = zr[0];
#pragma unroll
    for (int c = 1; c < REG; ++c)
      if (c < C) mx = fmaxf(mx, zr[c]);
    float er[REG > 0 ? REG : 1];
    float se = 0.f;
#pragma unroll
    for (int c = 0; c < REG; ++c)
      if (c < C) {
        er[c] = expf(zr[c] - mx);
        se += er[c];
      }
    const float ls = logf(se + 1e-12f);
#pragma unroll
    for (int c = 0; c < REG; ++c)
      if (c < C) {
        const float p = er[c] / se;
        sm[b + B * c] = p;
        row -= tr[c] * ((zr[c] - mx) - ls);
        float v = p - tr[c];
        if (mean) v *= inv_batch;
        g[b + B * c] = v;
      }
  } else if (REG == 0 && b < B) {
    float mx = z[b];
    for (int64_t c = 1; c < C; ++c) mx = fmaxf(mx, z[b + B * c]);
    float se = 0.f;
    for (int64_t c = 0; c < C; ++c) {
      const float e = expf(z[b + B * c] - mx);
      sm[b + B * c] = e;
      se += e;
    }
    const float ls = logf(se + 1e-12f);
    for (int64_t c = 0; c < C; ++c) {
      const float p = sm[b + B * c] / se;
      sm[b + B * c] = p;
      const float tv = t[b + B * c];
      row -= tv * ((z[b + B * c] - mx) - ls);
      float v = p - tv;
      if (mean) v *= inv_batch;
      g[b + B * c] = v;
    }
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) row += __shfl_xor(row, off, 64);
  if (lane == 0) smem[wave] = row;
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = 0.f;
    for (int w = 0; w < SCE_BLOCK / 64; ++w) s += smem[w];
    *loss = s / divisor;
  }
}

// softmax_ce_rows_kernel for C <= REG classes with the row in registers (all
// of a row's loads in flight at once) and, when g is given, the gradient of
// softmax_ce_backward_kernel written as well: the same arithmetic and the same
// per-block partials, in one pass.
template <int REG>
__global__ void __launch_bounds__(SCE_BLOCK) softmax_ce_rows_reg_kernel(
    const float* __restrict__ z, const float* __restrict__ t, float* __restrict__ sm,
    float* __restrict__ partial, float* __restrict__ g, int64_t B, int64_t C, int mean, float inv_batch) {
  __shared__ float smem[SCE_BLOCK / 64];
  float row = 0.f;
  const int64_t b = (int64_t)blockIdx.x * SCE_BLOCK + threadIdx.x;
  if (b < B) {
    float zr[REG], tr[REG], er[REG];
#pragma unroll
    for (int c = 0; c < REG; ++c) {
      zr[c] = c < C ? z[b + B * c] : 0.f;
      tr[c] = c < C ? t[b + B * c] : 0.f;
    }
    float mx = zr[0];
#pragma unroll
    for (int c = 1; c < REG; ++c)
      if (c < C) mx = fmaxf(mx, zr[c]);
    float se = 0.f;
#pragma unroll
    for (int c = 0; c < REG; ++c)
      if (c < C) {
        er[c] = expf(zr[c] - mx);
        se += er[c];
      }
    const float ls = logf(se + 1e-12f);
#pragma unroll
    for (int c = 0; c < REG; ++c)
      if (c < C) {
        const float p = er[c] / se;
        sm[b + B * c] = p;
        row -= tr[c] * ((zr[c] - mx) - ls);
        if (g) {
          float v = p - tr[c];
          if (mean) v *= inv_batch;
          g[b + B * c] = v;
        }
      }
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) row += __shfl_xor(row, off, 64);
  if (lane == 0) smem[wave] = row;
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = 0.f;
    for (int w = 0; w < SCE_BLOCK / 64; ++w) s += smem[w];
    partial[blockIdx.x] = s;
  }
}

__global__ void __launch_bounds__(RB) partial_sum_kernel(const float* __restrict__ partial,
                                                         int64_t count, float* __restrict__ out,
                                                         float divisor) {
  __shared__ float smem[RB / 64];
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < count; i += RB) s += partial[i];
  const float tot = block_sum(s, smem);
  if (threadIdx.x == 0) *out = tot / divisor;
}

__global__ void __launch_bounds__(256) softmax_ce_backward_kernel(const float* __restrict__ sm,
                                                                  const float* __restrict__ t,
                                                                  float* __restrict__ g, int64_t n,
                                                                  int mean, float inv_batch) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    float v = sm[i] - t[i];
    if (mean) v *= inv_batch;
    g[i] = v;
  }
}

int check_reduction(int reduction, const char* who) {
  CNHIP_REQUIRE(reduction == CNHIP_REDUCE_MEAN || reduction == CNHIP_REDUCE_SUM,
                "%s: reduction must be mean (0) or sum (1), got %d", who, reduction);
  return CNHIP_OK;
}

}  // namespace
}  // namespace cnhip

using cnhip::as_stream;

extern "C" {

int cnhip_relu_forward(const float* x, float* y, int64_t n, cnhip_stream_t s) {
  return cnhip::launch_unary<cnhip::ReluFwd>(x, y, n, as_stream(s), "cnhip_relu_forward");
}
int cnhip_relu_backward(const float* y, const float* dy, float* dx, int64_t n, cnhip_stream_t s) {
  return cnhip::launch_binary<cnhip::ReluBwd>(y, dy, dx, n, as_stream(s), "cnhip_relu_backward");
}
int cnhip_sigmoid_forward(const float* x, float* y, int64_t n, cnhip_stream_t s) {
  return cnhip::launch_unary<cnhip::SigmoidFwd>(x, y, n, as_stream(s), "cnhip_sigmoid_forward");
}
int cnhip_sigmoid_backward(const float* y, const float* dy, float* dx, int64_t n,
                           cnhip_stream_t s) {
  return cnhip::launch_binary<cnhip::SigmoidBwd>(y, dy, dx, n, as_stream(s),
                                                 "cnhip_sigmoid_backward");
}
int cnhip_tanh_forward(const float* x, float* y, int64_t n, cnhip_stream_t s) {
  return cnhip::launch_unary<cnhip::TanhFwd>(x, y, n, as_stream(s), "cnhip_tanh_forward");
}
int cnhip_tanh_backward(const float* y, const float* dy, float* dx, int64_t n, cnhip_stream_t s) {
  return cnhip::launch_binary<cnhip::TanhBwd>(y, dy, dx, n, as_stream(s), "cnhip_tanh_backward");
}

int cnhip_bce_forward(const float* pred, const float* target, float* loss, int64_t n,
                      int reduction, cnhip_stream_t s) {
  const char* who = "cnhip_bce_forward";
  CNHIP_TRY(cnhip::check_reduction(reduction, who));
  CNHIP_REQUIRE(n > 0, "%s: empty input", who);
  CNHIP_REQUIRE(pred && target && loss, "%s: NULL pointer", who);
  cnhip::HbmTimer timer("bce_forward_kernel", 8.0 * (double)n + 4.0, as_stream(s));
  hipLaunchKernelGGL(cnhip::bce_forward_kernel, dim3(1), dim3(cnhip::RB), 0, as_stream(s), pred,
                     target, loss, n, reduction);
  return cnhip::check_launch(who);
}

int cnhip_sigmoid_bce_head(const float* z, const float* target, float* p, float* loss, float* dz, int64_t n,
                           int loss_reduction, int grad_reduction, cnhip_stream_t s) {
  const char* who = "cnhip_sigmoid_bce_head";
  CNHIP_TRY(cnhip::check_reduction(loss_reduction, who));
  CNHIP_TRY(cnhip::check_reduction(grad_reduction, who));
  CNHIP_REQUIRE(n > 0, "%s: empty input", who);
  CNHIP_REQUIRE(z && target && p && loss && dz, "%s: NULL pointer", who);
  cnhip::HbmTimer timer("sigmoid_bce_head_kernel", 16.0 * (double)n + 4.0, as_stream(s));
  hipLaunchKernelGGL(cnhip::sigmoid_bce_head_kernel, dim3(1), dim3(cnhip::RB), 0, as_stream(s), z, target, p,
                     loss, dz, n, loss_reduction, grad_reduction);
  return cnhip::check_launch(who);
}

int cnhip_bce_backward(const float* pred, const float* target, float* grad, int64_t n,
                       int reduction, cnhip_stream_t s) {
  const char* who = "cnhip_bce_backward";
  CNHIP_TRY(cnhip::check_reduction(reduction, who));
  CNHIP_REQUIRE(n > 0, "%s: empty input", who);
  CNHIP_REQUIRE(pred && target && grad, "%s: NULL pointer", who);
  cnhip::HbmTimer timer("bce_backward_kernel", 12.0 * (double)n, as_stream(s));
  hipLaunchKernelGGL(cnhip::bce_backward_kernel, dim3(cnhip::elementwise_grid(n, 256)), dim3(256),
                     0, as_stream(s), pred, target, grad, n, reduction);
  return cnhip::check_launch(who);
}

int cnhip_mse_forward(const float* pred, const float* target, float* loss, int64_t n,
                      int reduction, cnhip_stream_t s) {
  const char* who = "cnhip_mse_forward";
  CNHIP_TRY(cnhip::check_reduction(reduction, who));
  CNHIP_REQUIRE(n > 0, "%s: empty input", who);
  CNHIP_REQUIRE(pred && target && loss, "%s: NULL pointer", who);
  cnhip::HbmTimer timer("mse_forward_kernel", 8.0 * (double)n + 4.0, as_stream(s));
  hipLaunchKernelGGL(cnhip::mse_forward_kernel, dim3(1), dim3(cnhip::RB), 0, as_stream(s), pred,
                     target, loss, n, reduction);
  return cnhip::check_launch(who);
}

int cnhip_mse_head(const float* pred, const float* target, float* loss, float* grad, int64_t n,
                   int loss_reduction, int grad_reduction, cnhip_stream_t s) {
  const char* who = "cnhip_mse_head";
  CNHIP_TRY(cnhip::check_reduction(loss_reduction, who));
  CNHIP_TRY(cnhip::check_reduction(grad_reduction, who));
  CNHIP_REQUIRE(n > 0, "%s: empty input", who);
  CNHIP_REQUIRE(pred && target && loss && grad, "%s: NULL pointer", who);
  const float scale = (grad_reduction == CNHIP_REDUCE_MEAN) ? 2.0f / (float)n : 2.0f;
  cnhip::HbmTimer timer("mse_head_kernel", 12.0 * (double)n + 4.0, as_stream(s));
  hipLaunchKernelGGL(cnhip::mse_head_kernel, dim3(1), dim3(cnhip::RB), 0, as_stream(s), pred, target, loss, grad,
                     n, loss_reduction, scale);
  return cnhip::check_launch(who);
}

int cnhip_mse_backward(const float* pred, const float* target, float* grad, int64_t n,
                       int reduction, cnhip_stream_t s) {
  const char* who = "cnhip_mse_backward";
  CNHIP_TRY(cnhip::check_reduction(reduction, who));
  CNHIP_REQUIRE(n > 0, "%s: empty input", who);
  CNHIP_REQUIRE(pred && target && grad, "%s: NULL pointer", who);
  const float scale = (reduction == CNHIP_REDUCE_MEAN) ? 2.0f / (float)n : 2.0f;
  cnhip::HbmTimer timer("mse_backward_kernel", 12.0 * (double)n, as_stream(s));
  hipLaunchKernelGGL(cnhip::mse_backward_kernel, dim3(cnhip::elementwise_grid(n, 256)), dim3(256),
                     0, as_stream(s), pred, target, grad, n, scale);
  return cnhip::check_launch(who);
}

namespace cnhip {
namespace {
// Softmax-CE over a batch of any size: per-block rows (+ the gradient when g
// is given) and partial losses, then partial_sum_kernel.  The two kernels
// give the same values; the register form serves rows of up to 32 classes.
int softmax_ce_multi(const float* logits, const float* targets, float* softmax_out, float* loss, float* g,
                     int64_t batch, int64_t classes, int reduction, hipStream_t st, const char* who) {
  const int64_t blocks = (batch + SCE_BLOCK - 1) / SCE_BLOCK;
  CNHIP_REQUIRE(blocks < ((int64_t)1 << 31), "%s: batch too large", who);
  void* ws = nullptr;
  CNHIP_TRY(scratch(st, kScratchLayer, (size_t)blocks * sizeof(float), &ws, who));
  float* partial = static_cast<float*>(ws);
  const int mean = reduction == CNHIP_REDUCE_MEAN ? 1 : 0;
  const float inv = 1.0f / (float)batch;
  {
    // logits and targets read, softmax (and the gradient) and the partials written
    HbmTimer timer("softmax_ce_rows_kernel", (g ? 16.0 : 12.0) * (double)batch * (double)classes + 4.0 * blocks,
                   st);
    if (classes <= 16)
      hipLaunchKernelGGL(softmax_ce_rows_reg_kernel<16>, dim3((unsigned)blocks), dim3(SCE_BLOCK), 0, st, logits,
                         targets, softmax_out, partial, g, batch, classes, mean, inv);
    else if (classes <= 32)
      hipLaunchKernelGGL(softmax_ce_rows_reg_kernel<32>, dim3((unsigned)blocks), dim3(SCE_BLOCK), 0, st, logits,
                         targets, softmax_out, partial, g, batch, classes, mean, inv);
    else
      hipLaunchKernelGGL(softmax_ce_rows_kernel, dim3((unsigned)blocks), dim3(SCE_BLOCK), 0, st, logits, targets,
                         softmax_out, partial, batch, classes);
    CNHIP_TRY(check_launch(who));
  }
  {
    // "mean" divides the summed loss by the batch size (softmax_cross_entropy.cpp:154-156)
    const float divisor = reduction == CNHIP_REDUCE_MEAN ? (float)batch : 1.0f;
    HbmTimer timer("partial_sum_kernel", 4.0 * blocks + 4.0, st);
    hipLaunchKernelGGL(partial_sum_kernel, dim3(1), dim3(RB), 0, st, partial, blocks, loss, divisor);
    CNHIP_TRY(check_launch(who));
  }
  if (g && classes > 32) {
    const int64_t n = batch * classes;
    HbmTimer timer("softmax_ce_backward_kernel", 12.0 * (double)n, st);
    hipLaunchKernelGGL(softmax_ce_backward_kernel, dim3(elementwise_grid(n, 256)), dim3(256), 0, st, softmax_out,
                       targets, g, n, mean, inv);
    CNHIP_TRY(check_launch(who));
  }
  return CNHIP_OK;
}
}  // namespace
}  // namespace cnhip

int cnhip_softmax_ce_forward(const float* logits, const float* targets, float* softmax_out,
                             float* loss, int64_t batch, int64_t classes, int reduction,
                             cnhip_stream_t s) {
  const char* who = "cnhip_softmax_ce_forward";
  CNHIP_TRY(cnhip::check_reduction(reduction, who));
  CNHIP_REQUIRE(batch > 0 && classes > 0, "%s: empty input", who);
  CNHIP_REQUIRE(logits && targets && softmax_out && loss, "%s: NULL pointer", who);
  return cnhip::softmax_ce_multi(logits, targets, softmax_out, loss, nullptr, batch, classes, reduction,
                                 as_stream(s), who);
}

int cnhip_softmax_ce_head(const float* logits, const float* targets, float* softmax_out, float* loss,
                          float* grad, int64_t batch, int64_t classes, int reduction, cnhip_stream_t s) {
  const char* who = "cnhip_softmax_ce_head";
  CNHIP_TRY(cnhip::check_reduction(reduction, who));
  CNHIP_REQUIRE(batch > 0 && classes > 0, "%s: empty input", who);
  CNHIP_REQUIRE(logits && targets && softmax_out && loss && grad, "%s: NULL pointer", who);
  if (batch > cnhip::SCE_BLOCK)
    return cnhip::softmax_ce_multi(logits, targets, softmax_out, loss, grad, batch, classes, reduction, as_stream(s),
                                   who);
  const float divisor = reduction == CNHIP_REDUCE_MEAN ? (float)batch : 1.0f;
  cnhip::HbmTimer timer("softmax_ce_head_kernel", 20.0 * (double)batch * (double)classes + 4.0, as_stream(s));
  const int mean = reduction == CNHIP_REDUCE_MEAN ? 1 : 0;
  const float inv = 1.0f / (float)batch;
  if (classes <= 16)
    hipLaunchKernelGGL(cnhip::softmax_ce_head_kernel<16>, dim3(1), dim3(cnhip::SCE_BLOCK), 0, as_stream(s),
                       logits, targets, softmax_out, loss, grad, batch, classes, divisor, mean, inv);
  else if (classes <= 32)
    hipLaunchKernelGGL(cnhip::softmax_ce_head_kernel<32>, dim3(1), dim3(cnhip::SCE_BLOCK), 0, as_stream(s),
                       logits, targets, softmax_out, loss, grad, batch, classes, divisor, mean, inv);
  else
    hipLaunchKernelGGL(cnhip::softmax_ce_head_kernel<0>, dim3(1), dim3(cnhip::SCE_BLOCK), 0, as_stream(s),
                       logits, targets, softmax_out, loss, grad, batch, classes, divisor, mean, inv);
  return cnhip::check_launch(who);
}

int cnhip_softmax_ce_backward(const float* softmax, const float* targets, float* grad,
                              int64_t batch, int64_t classes, int reduction, cnhip_stream_t s) {
  const char* who = "cnhip_softmax_ce_backward";
  CNHIP_TRY(cnhip::check_reduction(reduction, who));
  CNHIP_REQUIRE(batch > 0 && classes > 0, "%s: empty input", who);
  CNHIP_REQUIRE(softmax && targets && grad, "%s: NULL pointer", who);
  const int64_t n = batch * classes;
  const float inv_batch = 1.0f / (float)batch;
  cnhip::HbmTimer timer("softmax_ce_backward_kernel", 12.0 * (double)n, as_stream(s));
  hipLaunchKernelGGL(cnhip::softmax_ce_backward_kernel, dim3(cnhip::elementwise_grid(n, 256)),
                     dim3(256), 0, as_stream(s), softmax, targets, grad, n,
                     reduction == CNHIP_REDUCE_MEAN ? 1 : 0, inv_batch);
  return cnhip::check_launch(who);
}

}  // extern "C"
