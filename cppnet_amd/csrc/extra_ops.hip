// The reference's device ops off the BASELINE configs: LeakyReLU, Softmax,
// CategoricalCrossEntropy, MAE, Huber, Dropout, GlobalAvg/MaxPool2D and the
// SGD / Momentum / Adagrad / RMSProp updates.
//
// ref: activations/leacky_relu.cpp, activations/softmax.cpp,
// losses/categorical_cross_entropy.cpp, losses/mae.cpp, losses/huber.cpp,
// layers/dropout.cpp, layers/global_pool.cpp, optimizers/{sgd,momentum,
// adagrad,mrs_prop}.cpp (cpu-eigen / cpu semantics) and their gpu kernels
// (leaky_relu.cu, leaky_relu_grad.cu, categorical_ce.cu, mae.cu, huber.cu, dropout.cu,
// global_avg_pool2d.cu, global_max_pool2d.cu, sgd/momentum/adagrad/rmsprop
// step kernels).
//
// Layout is Eigen ColMajor.  Row-wise ops (softmax over the last dimension,
// the CCE rows, the global pools' (n, c) pairs) give one thread per row: the
// row index is the fastest-varying one in memory, so consecutive threads read
// consecutive addresses, and each thread runs its row's loop in the
// reference's order (the max scans and pooled sums are bit-identical to it).
// Elementwise parts and the optimizer updates evaluate the reference's
// expressions with one rounding per operation (no FMA contraction).
#include <hip/hip_runtime.h>

#include <cmath>

#include "common.hpp"

namespace cnhip {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int XB = 1024;  // single-block reductions

// Fixed-order sum over a 1024-thread block; valid on thread 0.
__device__ float xblock_sum(float v, float* smem) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  if (lane == 0) smem[wave] = v;
  __syncthreads();
  float r = 0.f;
  if (threadIdx.x == 0)
    for (int w = 0; w < XB / 64; ++w) r += smem[w];
  return r;
}

int check_reduce(int reduction, const char* who) {
  CNHIP_REQUIRE(reduction == CNHIP_REDUCE_MEAN || reduction == CNHIP_REDUCE_SUM,
                "%s: reduction must be mean (0) or sum (1), got %d", who, reduction);
  return CNHIP_OK;
}

// ---------------------------------------------------------------- LeakyReLU
// leacky_relu.cpp:93-156: y = x > 0 ? x : alpha x; dx = x > 0 ? dy : alpha dy
__global__ void __launch_bounds__(256) leaky_relu_fwd_kernel(const float* __restrict__ x,
                                                             float* __restrict__ y, int64_t n,
                                                             float alpha) {
#pragma clang fp contract(off)
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float v = x[i];
    y[i] = v > 0.0f ? v : alpha * v;
  }
}
__global__ void __launch_bounds__(256) leaky_relu_bwd_kernel(const float* __restrict__ x,
                                                             const float* __restrict__ dy,
                                                             float* __restrict__ dx, int64_t n,
                                                             float alpha) {
#pragma clang fp contract(off)
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    dx[i] = x[i] > 0.0f ? dy[i] : alpha * dy[i];
}

// ---------------------------------------------------------------- Softmax
// softmax.cpp:105-162 / 209-270 over the last dimension: element (r, j) at
// r + R*j; max from j = 0, exp(x - max) summed in j order, then divided.
__global__ void __launch_bounds__(256) softmax_last_fwd_kernel(const float* __restrict__ x,
                                                               float* __restrict__ y, int64_t R,
                                                               int64_t L) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= R) return;
  float mx = x[r];
  for (int64_t j = 1; j < L; ++j) mx = fmaxf(mx, x[r + R * j]);
  float s = 0.f;
  for (int64_t j = 0; j < L; ++j) {
    const float e = expf(x[r + R * j] - mx);
    y[r + R * j] = e;
    s += e;
  }
  for (int64_t j = 0; j < L; ++j) y[r + R * j] = y[r + R * j] / s;
}
// softmax.cpp:164-207 / 272-323: dot = sum_j dy y (j order); dx = y (dy - dot)
__global__ void __launch_bounds__(256) softmax_last_bwd_kernel(const float* __restrict__ y,
                                                               const float* __restrict__ dy,
                                                               float* __restrict__ dx, int64_t R,
                                                               int64_t L) {
#pragma clang fp contract(off)
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= R) return;
  float dot = 0.f;
  for (int64_t j = 0; j < L; ++j) dot += dy[r + R * j] * y[r + R * j];
  for (int64_t j = 0; j < L; ++j) dx[r + R * j] = y[r + R * j] * (dy[r + R * j] - dot);
}

// ---------------------------------------------------------------- CCE
// categorical_cross_entropy.cpp:167-259: one thread per row b of [B, C]:
// smoothed targets, softmax (from logits) or the given probabilities, and the
// row's loss sum_j -t log(clip(p)) into rowloss[b]; cce_sum_kernel adds the
// rows in a fixed order.
__global__ void __launch_bounds__(256) cce_rows_kernel(const float* __restrict__ pred,
                                                       const float* __restrict__ t,
                                                       float* __restrict__ probs,
                                                       float* __restrict__ tu,
                                                       float* __restrict__ rowloss, int64_t B,
                                                       int64_t C, int from_logits, float ls) {
#pragma clang fp contract(off)
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const float sf = ls / (float)C;
  for (int64_t j = 0; j < C; ++j) {
    const int64_t i = b + B * j;
    tu[i] = ls > 0.0f ? t[i] * (1.0f - ls) + sf : t[i];
  }
  if (from_logits) {
    float mx = pred[b];
    for (int64_t j = 1; j < C; ++j) mx = pred[b + B * j] > mx ? pred[b + B * j] : mx;
    float se = 0.f;
    for (int64_t j = 0; j < C; ++j) {
      const float e = expf(pred[b + B * j] - mx);
      probs[b + B * j] = e;
      se += e;
    }
    for (int64_t j = 0; j < C; ++j) probs[b + B * j] = probs[b + B * j] / se;
  } else {
    for (int64_t j = 0; j < C; ++j) probs[b + B * j] = pred[b + B * j];
  }
  const float eps = 1e-15f;
  float sample = 0.f;
  for (int64_t j = 0; j < C; ++j) {
    const float p = fmaxf(eps, fminf(1.0f - eps, probs[b + B * j]));
    sample -= tu[b + B * j] * logf(p);
  }
  rowloss[b] = sample;
}
__global__ void __launch_bounds__(XB) cce_sum_kernel(const float* __restrict__ rowloss, int64_t B,
                                                     float* __restrict__ loss, int mean) {
  __shared__ float smem[XB / 64];
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < B; i += XB) s += rowloss[i];
  const float tot = xblock_sum(s, smem);
  if (threadIdx.x == 0) *loss = mean ? tot / (float)B : tot;
}
// categorical_cross_entropy.cpp:316-380: g = p - t (logits) or -t / clip(p),
// then / B for "mean"
__global__ void __launch_bounds__(256) cce_bwd_kernel(const float* __restrict__ probs,
                                                      const float* __restrict__ tu,
                                                      float* __restrict__ g, int64_t n, int64_t B,
                                                      int from_logits, int mean) {
#pragma clang fp contract(off)
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const float eps = 1e-15f;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    float v;
    if (from_logits) {
      v = probs[i] - tu[i];
    } else {
      const float p = fmaxf(eps, fminf(1.0f - eps, probs[i]));
      v = -tu[i] / p;
    }
    g[i] = mean ? v / (float)B : v;
  }
}

// ---------------------------------------------------------------- MAE, Huber
// mae.cpp:102-160, huber.cpp:104-178
__global__ void __launch_bounds__(XB) mae_fwd_kernel(const float* __restrict__ p,
                                                     const float* __restrict__ t,
                                                     float* __restrict__ loss, int64_t n, int mean) {
  __shared__ float smem[XB / 64];
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += XB) s += fabsf(p[i] - t[i]);
  const float tot = xblock_sum(s, smem);
  if (threadIdx.x == 0) *loss = mean ? tot / (float)n : tot;
}
__global__ void __launch_bounds__(256) mae_bwd_kernel(const float* __restrict__ p,
                                                      const float* __restrict__ t,
                                                      float* __restrict__ g, int64_t n, float scale) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float d = p[i] - t[i];
    g[i] = d > 0.0f ? scale : (d < 0.0f ? -scale : 0.0f);
  }
}
__global__ void __launch_bounds__(XB) huber_fwd_kernel(const float* __restrict__ p,
                                                       const float* __restrict__ t,
                                                       float* __restrict__ loss, int64_t n,
                                                       float delta, int mean) {
#pragma clang fp contract(off)
  __shared__ float smem[XB / 64];
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += XB) {
    const float d = p[i] - t[i];
    const float a = fabsf(d);
    s += a <= delta ? 0.5f * d * d : delta * (a - 0.5f * delta);
  }
  const float tot = xblock_sum(s, smem);
  if (threadIdx.x == 0) *loss = mean ? tot / (float)n : tot;
}
__global__ void __launch_bounds__(256) huber_bwd_kernel(const float* __restrict__ p,
                                                        const float* __restrict__ t,
                                                        float* __restrict__ g, int64_t n,
                                                        float delta, float scale) {
#pragma clang fp contract(off)
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float d = p[i] - t[i];
    g[i] = fabsf(d) <= delta ? scale * d : scale * delta * (d > 0.0f ? 1.0f : -1.0f);
  }
}

// ---------------------------------------------------------------- Dropout
// dropout.cpp:140-270: out = x * mask * scale with mask ~ Bernoulli(1 - p).
// The reference draws the mask on the host from a time-seeded mt19937
// (dropout.cpp:19-21); here it comes from a counter-based generator: entry
// i of a call keeps its input when u(seed, offset + i) < 1 - p, with
// u = (top 24 bits of splitmix64(seed + (offset + i) * golden)) / 2^24, so a
// mask is reproducible from (seed, offset) and needs no state.
__device__ __forceinline__ float dropout_u(uint64_t seed, uint64_t idx) {
  uint64_t z = seed + idx * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z ^= z >> 31;
  return (float)(z >> 40) * (1.0f / 16777216.0f);
}
__global__ void __launch_bounds__(256) dropout_fwd_kernel(const float* __restrict__ x,
                                                          float* __restrict__ y,
                                                          uint8_t* __restrict__ mask, int64_t n,
                                                          float keep, float scale, uint64_t seed,
                                                          uint64_t offset) {
#pragma clang fp contract(off)
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint8_t m = dropout_u(seed, offset + (uint64_t)i) < keep ? 1 : 0;
    mask[i] = m;
    y[i] = x[i] * (float)m * scale;
  }
}
__global__ void __launch_bounds__(256) dropout_bwd_kernel(const float* __restrict__ dy,
                                                          const uint8_t* __restrict__ mask,
                                                          float* __restrict__ dx, int64_t n,
                                                          float scale) {
#pragma clang fp contract(off)
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    dx[i] = dy[i] * (float)mask[i] * scale;
}

// ---------------------------------------------------------------- global pools
// global_pool.cpp:111-159: per (n, c), sum over h (outer), w (inner) in order,
// times 1 / (H W).  Thread per q = n + N*c; input (n, c, h, w) at
// q + N*C*(h + H*w).
__global__ void __launch_bounds__(256) gavg_fwd_kernel(const float* __restrict__ X,
                                                       float* __restrict__ Y, int64_t NC, int64_t H,
                                                       int64_t W, float inv) {
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= NC) return;
  float s = 0.f;
  for (int64_t h = 0; h < H; ++h)
    for (int64_t w = 0; w < W; ++w) s += X[q + NC * (h + H * w)];
  Y[q] = s * inv;
}
// global_pool.cpp:161-210: every input of (n, c) gets dY(n, c) * inv
__global__ void __launch_bounds__(256) gavg_bwd_kernel(const float* __restrict__ dY,
                                                       float* __restrict__ dX, int64_t NC,
                                                       int64_t total, float inv) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride)
    dX[i] = dY[i % NC] * inv;
}
// global_pool.cpp:305-373: strict > scan from -inf, h outer, w inner
__global__ void __launch_bounds__(256) gmax_fwd_kernel(const float* __restrict__ X,
                                                       float* __restrict__ Y,
                                                       int32_t* __restrict__ ah,
                                                       int32_t* __restrict__ aw, int64_t NC,
                                                       int64_t H, int64_t W) {
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= NC) return;
  float mx = -INFINITY;
  int32_t bh = 0, bw = 0;
  for (int64_t h = 0; h < H; ++h)
    for (int64_t w = 0; w < W; ++w) {
      const float v = X[q + NC * (h + H * w)];
      if (v > mx) {
        mx = v;
        bh = (int32_t)h;
        bw = (int32_t)w;
      }
    }
  Y[q] = mx;
  ah[q] = bh;
  aw[q] = bw;
}
// global_pool.cpp:375-395: dX is dY(n, c) at the argmax, 0 elsewhere; every
// element written, no atomics
__global__ void __launch_bounds__(256) gmax_bwd_kernel(const float* __restrict__ dY,
                                                       const int32_t* __restrict__ ah,
                                                       const int32_t* __restrict__ aw,
                                                       float* __restrict__ dX, int64_t NC,
                                                       int64_t H, int64_t total) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t q = i % NC, hw = i / NC;
    const int64_t h = hw % H, w = hw / H;
    dX[i] = (h == ah[q] && w == aw[q]) ? dY[q] : 0.0f;
  }
}

// ---------------------------------------------------------------- optimizers
// One launch updates up to 64 tensors; a block owns OPT_CHUNK consecutive
// parameters of one tensor.
//   SGD      (sgd.cpp:54-68)       W -= lr g
//   Momentum (momentum.cpp:81-104) v = mu v - lr g; W += v
//   Adagrad  (adagrad.cpp:83-106)  a += g g; W -= lr g / (sqrt(a) + eps)
//   RMSProp  (mrs_prop.cpp:83-106) s = rho s + (1 - rho) g g; W -= lr g / (sqrt(s) + eps)
constexpr int OPT_MAX = 64;
constexpr int OPT_BLOCK = 256;
constexpr int OPT_CHUNK = OPT_BLOCK * 8;

struct OptTensor {
  float* W;
  const float* g;
  float* s;  // velocity / accumulator / mean square (unused for SGD)
  int64_t n;
  int first_block;
};
struct OptBatch {
  OptTensor t[OPT_MAX];
  int count;
};

template <int KIND>
__device__ __forceinline__ void opt_one(float& w, float g, float& s, float lr, float h, float eps) {
#pragma clang fp contract(off)
  if (KIND == CNHIP_OPT_SGD) {
    w -= lr * g;
  } else if (KIND == CNHIP_OPT_MOMENTUM) {
    s = h * s - lr * g;
    w += s;
  } else if (KIND == CNHIP_OPT_ADAGRAD) {
    s += g * g;
    w -= lr * g / (sqrtf(s) + eps);
  } else {
    s = h * s + (1.0f - h) * g * g;
    w -= lr * g / (sqrtf(s) + eps);
  }
}

template <int KIND>
__global__ void __launch_bounds__(OPT_BLOCK) opt_multi_kernel(OptBatch batch, float lr, float h, float eps,
                                                               UpdateGuard guard) {
  if (update_withheld(guard)) return;
  int ti = 0;
  for (int i = 1; i < batch.count; ++i)
    if ((int)blockIdx.x >= batch.t[i].first_block) ti = i;
  const OptTensor& T = batch.t[ti];
  const int64_t begin = (int64_t)((int)blockIdx.x - T.first_block) * OPT_CHUNK;
#pragma unroll
  for (int r = 0; r < OPT_CHUNK / OPT_BLOCK; ++r) {
    const int64_t i = begin + (int64_t)r * OPT_BLOCK + threadIdx.x;
    if (i < T.n) {
      float w = T.W[i], s = KIND == CNHIP_OPT_SGD ? 0.f : T.s[i];
      opt_one<KIND>(w, T.g[i], s, lr, h, eps);
      T.W[i] = w;
      if (KIND != CNHIP_OPT_SGD) T.s[i] = s;
    }
  }
}

}  // namespace
}  // namespace cnhip

using cnhip::as_stream;

extern "C" {

int cnhip_leaky_relu_forward(const float* x, float* y, int64_t n, float alpha, cnhip_stream_t s) {
  const char* who = "cnhip_leaky_relu_forward";
  CNHIP_REQUIRE(n >= 0, "%s: negative size", who);
  if (n == 0) return CNHIP_OK;
  CNHIP_REQUIRE(x && y, "%s: NULL pointer", who);
  cnhip::HbmTimer timer("leaky_relu_fwd_kernel", 8.0 * (double)n, as_stream(s));
  hipLaunchKernelGGL(cnhip::leaky_relu_fwd_kernel, dim3(cnhip::elementwise_grid(n, 256)), dim3(256), 0,
                     as_stream(s), x, y, n, alpha);
  return cnhip::check_launch(who);
}

int cnhip_leaky_relu_backward(const float* x, const float* dy, float* dx, int64_t n, float alpha,
                              cnhip_stream_t s) {
  const char* who = "cnhip_leaky_relu_backward";
  CNHIP_REQUIRE(n >= 0, "%s: negative size", who);
  if (n == 0) return CNHIP_OK;
  CNHIP_REQUIRE(x && dy && dx, "%s: NULL pointer", who);
  cnhip::HbmTimer timer("leaky_relu_bwd_kernel", 12.0 * (double)n, as_stream(s));
  hipLaunchKernelGGL(cnhip::leaky_relu_bwd_kernel, dim3(cnhip::elementwise_grid(n, 256)), dim3(256), 0,
                     as_stream(s), x, dy, dx, n, alpha);
  return cnhip::check_launch(who);
}

int cnhip_softmax_forward(const float* x, float* y, int64_t rows, int64_t len, cnhip_stream_t s) {
  const char* who = "cnhip_softmax_forward";
  CNHIP_REQUIRE(rows > 0 && len > 0, "%s: empty input (rows=%lld len=%lld)", who, (long long)rows,
                (long long)len);
  CNHIP_REQUIRE(x && y && x != y, "%s: NULL or aliased pointers", who);
  cnhip::HbmTimer timer("softmax_last_fwd_kernel", 8.0 * (double)rows * (double)len, as_stream(s));
  hipLaunchKernelGGL(cnhip::softmax_last_fwd_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0,
                     as_stream(s), x, y, rows, len);
  return cnhip::check_launch(who);
}

int cnhip_softmax_backward(const float* y, const float* dy, float* dx, int64_t rows, int64_t len,
                           cnhip_stream_t s) {
  const char* who = "cnhip_softmax_backward";
  CNHIP_REQUIRE(rows > 0 && len > 0, "%s: empty input", who);
  CNHIP_REQUIRE(y && dy && dx && dx != y && dx != dy, "%s: NULL or aliased pointers", who);
  cnhip::HbmTimer timer("softmax_last_bwd_kernel", 12.0 * (double)rows * (double)len, as_stream(s));
  hipLaunchKernelGGL(cnhip::softmax_last_bwd_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0,
                     as_stream(s), y, dy, dx, rows, len);
  return cnhip::check_launch(who);
}

int cnhip_cce_forward(const float* pred, const float* targets, float* probs, float* targets_used,
                      float* loss, int64_t B, int64_t C, int from_logits, float label_smoothing,
                      int reduction, cnhip_stream_t s) {
  const char* who = "cnhip_cce_forward";
  CNHIP_TRY(cnhip::check_reduce(reduction, who));
  CNHIP_REQUIRE(B > 0 && C > 0, "%s: empty input", who);
  CNHIP_REQUIRE(pred && targets && probs && targets_used && loss, "%s: NULL pointer", who);
  CNHIP_REQUIRE(label_smoothing >= 0.0f && label_smoothing <= 1.0f, "%s: label_smoothing %g outside [0, 1]",
                who, (double)label_smoothing);
  hipStream_t st = as_stream(s);
  void* ws = nullptr;
  CNHIP_TRY(cnhip::scratch(st, cnhip::kScratchLayer, (size_t)B * sizeof(float), &ws, who));
  float* rowloss = static_cast<float*>(ws);
  {
    cnhip::HbmTimer timer("cce_rows_kernel", 16.0 * (double)B * (double)C, st);
    hipLaunchKernelGGL(cnhip::cce_rows_kernel, dim3((unsigned)((B + 255) / 256)), dim3(256), 0, st, pred,
                       targets, probs, targets_used, rowloss, B, C, from_logits ? 1 : 0, label_smoothing);
    CNHIP_TRY(cnhip::check_launch(who));
  }
  hipLaunchKernelGGL(cnhip::cce_sum_kernel, dim3(1), dim3(cnhip::XB), 0, st, rowloss, B, loss,
                     reduction == CNHIP_REDUCE_MEAN ? 1 : 0);
  return cnhip::check_launch(who);
}

int cnhip_cce_backward(const float* probs, const float* targets_used, float* grad, int64_t B, int64_t C,
                       int from_logits, int reduction, cnhip_stream_t s) {
  const char* who = "cnhip_cce_backward";
  CNHIP_TRY(cnhip::check_reduce(reduction, who));
  CNHIP_REQUIRE(B > 0 && C > 0, "%s: empty input", who);
  CNHIP_REQUIRE(probs && targets_used && grad, "%s: NULL pointer", who);
  const int64_t n = B * C;
  cnhip::HbmTimer timer("cce_bwd_kernel", 12.0 * (double)n, as_stream(s));
  hipLaunchKernelGGL(cnhip::cce_bwd_kernel, dim3(cnhip::elementwise_grid(n, 256)), dim3(256), 0, as_stream(s),
                     probs, targets_used, grad, n, B, from_logits ? 1 : 0,
                     reduction == CNHIP_REDUCE_MEAN ? 1 : 0);
  return cnhip::check_launch(who);
}

int cnhip_mae_forward(const float* p, const float* t, float* loss, int64_t n, int reduction,
                      cnhip_stream_t s) {
  const char* who = "cnhip_mae_forward";
  CNHIP_TRY(cnhip::check_reduce(reduction, who));
  CNHIP_REQUIRE(n > 0, "%s: empty input", who);
  CNHIP_REQUIRE(p && t && loss, "%s: NULL pointer", who);
  hipLaunchKernelGGL(cnhip::mae_fwd_kernel, dim3(1), dim3(cnhip::XB), 0, as_stream(s), p, t, loss, n,
                     reduction == CNHIP_REDUCE_MEAN ? 1 : 0);
  return cnhip::check_launch(who);
}

int cnhip_mae_backward(const float* p, const float* t, float* g, int64_t n, int reduction,
                       cnhip_stream_t s) {
  const char* who = "cnhip_mae_backward";
  CNHIP_TRY(cnhip::check_reduce(reduction, who));
  CNHIP_REQUIRE(n > 0, "%s: empty input", who);
  CNHIP_REQUIRE(p && t && g, "%s: NULL pointer", who);
  const float scale = reduction == CNHIP_REDUCE_MEAN ? 1.0f / (float)n : 1.0f;
  hipLaunchKernelGGL(cnhip::mae_bwd_kernel, dim3(cnhip::elementwise_grid(n, 256)), dim3(256), 0, as_stream(s),
                     p, t, g, n, scale);
  return cnhip::check_launch(who);
}

int cnhip_huber_forward(const float* p, const float* t, float* loss, int64_t n, float delta,
                        int reduction, cnhip_stream_t s) {
  const char* who = "cnhip_huber_forward";
  CNHIP_TRY(cnhip::check_reduce(reduction, who));
  CNHIP_REQUIRE(n > 0, "%s: empty input", who);
  CNHIP_REQUIRE(p && t && loss, "%s: NULL pointer", who);
  hipLaunchKernelGGL(cnhip::huber_fwd_kernel, dim3(1), dim3(cnhip::XB), 0, as_stream(s), p, t, loss, n, delta,
                     reduction == CNHIP_REDUCE_MEAN ? 1 : 0);
  return cnhip::check_launch(who);
}

int cnhip_huber_backward(const float* p, const float* t, float* g, int64_t n, float delta, int reduction,
                         cnhip_stream_t s) {
  const char* who = "cnhip_huber_backward";
  CNHIP_TRY(cnhip::check_reduce(reduction, who));
  CNHIP_REQUIRE(n > 0, "%s: empty input", who);
  CNHIP_REQUIRE(p && t && g, "%s: NULL pointer", who);
  const float scale = reduction == CNHIP_REDUCE_MEAN ? 1.0f / (float)n : 1.0f;
  hipLaunchKernelGGL(cnhip::huber_bwd_kernel, dim3(cnhip::elementwise_grid(n, 256)), dim3(256), 0,
                     as_stream(s), p, t, g, n, delta, scale);
  return cnhip::check_launch(who);
}

int cnhip_dropout_forward(const float* x, float* y, uint8_t* mask, int64_t n, float p, uint64_t seed,
                          uint64_t offset, cnhip_stream_t s) {
  const char* who = "cnhip_dropout_forward";
  CNHIP_REQUIRE(n >= 0, "%s: negative size", who);
  CNHIP_REQUIRE(p >= 0.0f && p < 1.0f, "%s: drop probability %g outside [0, 1)", who, (double)p);
  if (n == 0) return CNHIP_OK;
  CNHIP_REQUIRE(x && y && mask, "%s: NULL pointer", who);
  const float scale = 1.0f / (1.0f - p);  // dropout.cpp:17
  cnhip::HbmTimer timer("dropout_fwd_kernel", 9.0 * (double)n, as_stream(s));
  hipLaunchKernelGGL(cnhip::dropout_fwd_kernel, dim3(cnhip::elementwise_grid(n, 256)), dim3(256), 0,
                     as_stream(s), x, y, mask, n, 1.0f - p, scale, seed, offset);
  return cnhip::check_launch(who);
}

int cnhip_dropout_backward(const float* dy, const uint8_t* mask, float* dx, int64_t n, float p,
                           cnhip_stream_t s) {
  const char* who = "cnhip_dropout_backward";
  CNHIP_REQUIRE(n >= 0, "%s: negative size", who);
  CNHIP_REQUIRE(p >= 0.0f && p < 1.0f, "%s: drop probability %g outside [0, 1)", who, (double)p);
  if (n == 0) return CNHIP_OK;
  CNHIP_REQUIRE(dy && mask && dx, "%s: NULL pointer", who);
  const float scale = 1.0f / (1.0f - p);
  cnhip::HbmTimer timer("dropout_bwd_kernel", 9.0 * (double)n, as_stream(s));
  hipLaunchKernelGGL(cnhip::dropout_bwd_kernel, dim3(cnhip::elementwise_grid(n, 256)), dim3(256), 0,
                     as_stream(s), dy, mask, dx, n, scale);
  return cnhip::check_launch(who);
}

int cnhip_global_avgpool_forward(const float* X, float* Y, int64_t N, int64_t C, int64_t H, int64_t W,
                                 cnhip_stream_t s) {
  const char* who = "cnhip_global_avgpool_forward";
  CNHIP_REQUIRE(N > 0 && C > 0 && H > 0 && W > 0, "%s: bad shape", who);
  CNHIP_REQUIRE(X && Y, "%s: NULL pointer", who);
  const int64_t NC = N * C;
  const float inv = 1.0f / (float)(H * W);
  cnhip::HbmTimer timer("gavg_fwd_kernel", 4.0 * (double)NC * (double)(H * W + 1), as_stream(s));
  hipLaunchKernelGGL(cnhip::gavg_fwd_kernel, dim3((unsigned)((NC + 255) / 256)), dim3(256), 0, as_stream(s), X,
                     Y, NC, H, W, inv);
  return cnhip::check_launch(who);
}

int cnhip_global_avgpool_backward(const float* dY, float* dX, int64_t N, int64_t C, int64_t H, int64_t W,
                                  cnhip_stream_t s) {
  const char* who = "cnhip_global_avgpool_backward";
  CNHIP_REQUIRE(N > 0 && C > 0 && H > 0 && W > 0, "%s: bad shape", who);
  CNHIP_REQUIRE(dY && dX, "%s: NULL pointer", who);
  const int64_t NC = N * C, total = NC * H * W;
  const float inv = 1.0f / (float)(H * W);
  cnhip::HbmTimer timer("gavg_bwd_kernel", 4.0 * (double)(total + NC), as_stream(s));
  hipLaunchKernelGGL(cnhip::gavg_bwd_kernel, dim3(cnhip::elementwise_grid(total, 256)), dim3(256), 0,
                     as_stream(s), dY, dX, NC, total, inv);
  return cnhip::check_launch(who);
}

int cnhip_global_maxpool_forward(const float* X, float* Y, int32_t* argmax_h, int32_t* argmax_w, int64_t N,
                                 int64_t C, int64_t H, int64_t W, cnhip_stream_t s) {
  const char* who = "cnhip_global_maxpool_forward";
  CNHIP_REQUIRE(N > 0 && C > 0 && H > 0 && W > 0, "%s: bad shape", who);
  CNHIP_REQUIRE(H < ((int64_t)1 << 31) && W < ((int64_t)1 << 31), "%s: spatial size too large", who);
  CNHIP_REQUIRE(X && Y && argmax_h && argmax_w, "%s: NULL pointer", who);
  const int64_t NC = N * C;
  cnhip::HbmTimer timer("gmax_fwd_kernel", 4.0 * (double)NC * (double)(H * W + 3), as_stream(s));
  hipLaunchKernelGGL(cnhip::gmax_fwd_kernel, dim3((unsigned)((NC + 255) / 256)), dim3(256), 0, as_stream(s), X,
                     Y, argmax_h, argmax_w, NC, H, W);
  return cnhip::check_launch(who);
}

int cnhip_global_maxpool_backward(const float* dY, const int32_t* argmax_h, const int32_t* argmax_w,
                                  float* dX, int64_t N, int64_t C, int64_t H, int64_t W, cnhip_stream_t s) {
  const char* who = "cnhip_global_maxpool_backward";
  CNHIP_REQUIRE(N > 0 && C > 0 && H > 0 && W > 0, "%s: bad shape", who);
  CNHIP_REQUIRE(dY && argmax_h && argmax_w && dX, "%s: NULL pointer", who);
  const int64_t NC = N * C, total = NC * H * W;
  cnhip::HbmTimer timer("gmax_bwd_kernel", 4.0 * (double)total + 12.0 * (double)NC, as_stream(s));
  hipLaunchKernelGGL(cnhip::gmax_bwd_kernel, dim3(cnhip::elementwise_grid(total, 256)), dim3(256), 0,
                     as_stream(s), dY, argmax_h, argmax_w, dX, NC, H, total);
  return cnhip::check_launch(who);
}

int cnhip_optimizer_step_multi(int kind, int count, float* const* W, const float* const* g,
                               float* const* state, const int64_t* n, float lr, float hyper, float eps,
                               cnhip_stream_t s) {
  const char* who = "cnhip_optimizer_step_multi";
  CNHIP_REQUIRE(kind >= CNHIP_OPT_SGD && kind <= CNHIP_OPT_RMSPROP, "%s: unknown optimizer kind %d", who,
                kind);
  CNHIP_REQUIRE(count >= 0 && count <= cnhip::OPT_MAX, "%s: count %d outside [0, %d]", who, count,
                cnhip::OPT_MAX);
  if (count == 0) return CNHIP_OK;
  CNHIP_REQUIRE(W && g && n && (kind == CNHIP_OPT_SGD || state), "%s: NULL host array", who);
  cnhip::OptBatch b;
  b.count = count;
  int blocks = 0;
  double params = 0.0;
  for (int i = 0; i < count; ++i) {
    CNHIP_REQUIRE(n[i] >= 0, "%s: negative size", who);
    CNHIP_REQUIRE(n[i] == 0 || (W[i] && g[i] && (kind == CNHIP_OPT_SGD || state[i])), "%s: NULL pointer", who);
    b.t[i] = cnhip::OptTensor{W[i], g[i], kind == CNHIP_OPT_SGD ? nullptr : state[i], n[i], blocks};
    const int64_t nb = (n[i] + cnhip::OPT_CHUNK - 1) / cnhip::OPT_CHUNK;
    CNHIP_REQUIRE(blocks + nb < ((int64_t)1 << 30), "%s: too many parameters", who);
    blocks += (int)nb;
    params += (double)n[i];
  }
  if (blocks == 0) return CNHIP_OK;
  hipStream_t st = as_stream(s);
  cnhip::UpdateGuard guard;
  CNHIP_TRY(cnhip::update_guard(&guard, who));
  // W and g read, W written; the state read and written (not for SGD)
  cnhip::HbmTimer timer("opt_multi_kernel", (kind == CNHIP_OPT_SGD ? 12.0 : 20.0) * params, st);
  switch (kind) {
    case CNHIP_OPT_SGD:
      hipLaunchKernelGGL(cnhip::opt_multi_kernel<CNHIP_OPT_SGD>, dim3(blocks), dim3(cnhip::OPT_BLOCK), 0, st, b,
                         lr, hyper, eps, guard);
      break;
    case CNHIP_OPT_MOMENTUM:
      hipLaunchKernelGGL(cnhip::opt_multi_kernel<CNHIP_OPT_MOMENTUM>, dim3(blocks), dim3(cnhip::OPT_BLOCK), 0,
                         st, b, lr, hyper, eps, guard);
      break;
    case CNHIP_OPT_ADAGRAD:
      hipLaunchKernelGGL(cnhip::opt_multi_kernel<CNHIP_OPT_ADAGRAD>, dim3(blocks), dim3(cnhip::OPT_BLOCK), 0,
                         st, b, lr, hyper, eps, guard);
      break;
    default:
      hipLaunchKernelGGL(cnhip::opt_multi_kernel<CNHIP_OPT_RMSPROP>, dim3(blocks), dim3(cnhip::OPT_BLOCK), 0,
                         st, b, lr, hyper, eps, guard);
      break;
  }
  return cnhip::check_launch(who);
}

}  // extern "C"
