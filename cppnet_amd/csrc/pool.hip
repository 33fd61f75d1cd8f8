// MaxPool2D forward (value + int32 window-local argmax) and backward.
//
// ref: MaxPool2D::forward/backward, src/CppNet/layers/max_pool2d.cpp:32-131
// (semantics: HO = (H - pool)/stride + 1, no padding; argmax = ph*pool + pw
// of the FIRST maximum, strict >, search from -inf; backward adds dY at the
// argmax into a zeroed dX) and maxpool2d_forward.cu / maxpool2d_backward.cu
// (the reference gpu path, which starts from -FLT_MAX and scatters with
// atomicAdd after a memset).
//
// ColMajor [N, C, H, W] puts the batch index fastest: one thread per output
// (forward) or per input element (backward) with n = thread index gives
// coalesced reads of every window tap.  The backward is a gather: each input
// element sums dY over the windows that contain it and picked it, so no
// atomics and no separate zero-fill are needed, and non-overlapping windows
// (stride == pool) produce exactly one term per element.
#include <hip/hip_runtime.h>

#include <cmath>

#include "common.hpp"

namespace cnhip {
namespace {

struct PoolDims {
  int64_t N, C, H, W, pool, stride, HO, WO;
};

__global__ void __launch_bounds__(256) maxpool_fwd_kernel(PoolDims d, const float* __restrict__ X,
                                                          float* __restrict__ Y,
                                                          int32_t* __restrict__ idx) {
  const int64_t total = d.N * d.C * d.HO * d.WO;
  for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < total;
       o += (int64_t)gridDim.x * blockDim.x) {
    // o = n + N*(c + C*(oh + HO*ow))
    const int64_t n = o % d.N;
    int64_t r = o / d.N;
    const int64_t c = r % d.C;
    r /= d.C;
    const int64_t oh = r % d.HO, ow = r / d.HO;
    float mx = -INFINITY;
    int32_t mi = 0;
    for (int64_t ph = 0; ph < d.pool; ++ph)
      for (int64_t pw = 0; pw < d.pool; ++pw) {
        const int64_t ih = oh * d.stride + ph, iw = ow * d.stride + pw;
        const float v = X[n + d.N * (c + d.C * (ih + d.H * iw))];
        if (v > mx) {
          mx = v;
          mi = (int32_t)(ph * d.pool + pw);
        }
      }
    Y[o] = mx;
    idx[o] = mi;
  }
}

__global__ void __launch_bounds__(256) maxpool_bwd_kernel(PoolDims d, const float* __restrict__ dY,
                                                          const int32_t* __restrict__ idx,
                                                          float* __restrict__ dX) {
  const int64_t total = d.N * d.C * d.H * d.W;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = i % d.N;
    int64_t r = i / d.N;
    const int64_t c = r % d.C;
    r /= d.C;
    const int64_t ih = r % d.H, iw = r / d.H;
    // windows (oh, ow) with oh*stride <= ih < oh*stride + pool
    const int64_t oh_lo = ih >= d.pool ? (ih - d.pool) / d.stride + 1 : 0;
    const int64_t oh_hi = min(ih / d.stride, d.HO - 1);
    const int64_t ow_lo = iw >= d.pool ? (iw - d.pool) / d.stride + 1 : 0;
    const int64_t ow_hi = min(iw / d.stride, d.WO - 1);
    float g = 0.f;
    for (int64_t oh = oh_lo; oh <= oh_hi; ++oh)
      for (int64_t ow = ow_lo; ow <= ow_hi; ++ow) {
        const int32_t want = (int32_t)((ih - oh * d.stride) * d.pool + (iw - ow * d.stride));
        const int64_t o = n + d.N * (c + d.C * (oh + d.HO * ow));
        if (idx[o] == want) g += dY[o];
      }
    dX[i] = g;
  }
}

int pool_dims(PoolDims& d, int64_t N, int64_t C, int64_t H, int64_t W, int64_t pool,
              int64_t stride, const char* who) {
  CNHIP_REQUIRE(N > 0 && C > 0 && H > 0 && W > 0 && pool > 0,
                "%s: bad shape N=%lld C=%lld H=%lld W=%lld pool=%lld", who, (long long)N,
                (long long)C, (long long)H, (long long)W, (long long)pool);
  if (stride <= 0) stride = pool;  // max_pool2d.cpp:25-28: stride defaults to pool
  CNHIP_REQUIRE(pool <= H && pool <= W, "%s: pool %lld larger than the input %lldx%lld", who,
                (long long)pool, (long long)H, (long long)W);
  d = PoolDims{N, C, H, W, pool, stride, (H - pool) / stride + 1, (W - pool) / stride + 1};
  return CNHIP_OK;
}

}  // namespace
}  // namespace cnhip

extern "C" {

int cnhip_maxpool2d_forward(const float* X, float* Y, int32_t* idx, int64_t N, int64_t C,
                            int64_t H, int64_t W, int64_t pool, int64_t stride,
                            cnhip_stream_t stream) {
  const char* who = "cnhip_maxpool2d_forward";
  cnhip::PoolDims d;
  CNHIP_TRY(cnhip::pool_dims(d, N, C, H, W, pool, stride, who));
  CNHIP_REQUIRE(X && Y && idx, "%s: NULL pointer", who);
  const int64_t total = N * C * d.HO * d.WO;
  hipLaunchKernelGGL(cnhip::maxpool_fwd_kernel, dim3(cnhip::elementwise_grid(total, 256)),
                     dim3(256), 0, cnhip::as_stream(stream), d, X, Y, idx);
  return cnhip::check_launch(who);
}

int cnhip_maxpool2d_backward(const float* dY, const int32_t* idx, float* dX, int64_t N, int64_t C,
                             int64_t H, int64_t W, int64_t pool, int64_t stride,
                             cnhip_stream_t stream) {
  const char* who = "cnhip_maxpool2d_backward";
  cnhip::PoolDims d;
  CNHIP_TRY(cnhip::pool_dims(d, N, C, H, W, pool, stride, who));
  CNHIP_REQUIRE(dY && idx && dX, "%s: NULL pointer", who);
  const int64_t total = N * C * H * W;
  hipLaunchKernelGGL(cnhip::maxpool_bwd_kernel, dim3(cnhip::elementwise_grid(total, 256)),
                     dim3(256), 0, cnhip::as_stream(stream), d, dY, idx, dX);
  return cnhip::check_launch(who);
}

}  // extern "C"
