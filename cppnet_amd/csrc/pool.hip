// MaxPool2D forward (value + int32 window-local argmax) and backward.
//
// ref: MaxPool2D::forward/backward, src/CppNet/layers/max_pool2d.cpp:32-131
// (semantics: HO = (H - pool)/stride + 1, no padding; argmax = ph*pool + pw
// of the FIRST maximum, strict >, search from -inf; backward adds dY at the
// argmax into a zeroed dX) and maxpool2d_forward.cu / maxpool2d_backward.cu
// (the reference gpu path, which starts from -FLT_MAX and scatters with
// atomicAdd after a memset).
//
// ColMajor [N, C, H, W] puts the batch index fastest: blocks own window
// positions and their threads run over n, so every window tap is a coalesced
// read.  The backward writes every element of dX itself, with no atomics and
// no separate zero-fill: as a gather over the windows containing an input
// element in general, and as one block per window when the windows tile the
// input exactly (each element then gets exactly one term).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <type_traits>
#include <utility>

#include "act_math.hpp"
#include "common.hpp"

namespace cnhip {
namespace {

struct PoolDims {
  int64_t N, C, H, W, pool, stride, HO, WO;
};

// Blocks loop over positions (c + C*(h + H*w)) from a grid capped at
// kPoolGrid: the position is decoded once per iteration in 32-bit integers
// (every position count here is < 2^31), and the block's threads stride over
// the batch index n, contiguous in memory, so each window tap is one
// coalesced read.
constexpr int kPoolGrid = 4096;

__global__ void __launch_bounds__(256) maxpool_fwd_kernel(PoolDims d, const float* __restrict__ X,
                                                          float* __restrict__ Y,
                                                          int32_t* __restrict__ idx) {
  const int C = (int)d.C, HO = (int)d.HO, pool = (int)d.pool, stride = (int)d.stride;
  const int positions = C * HO * (int)d.WO;
  const int64_t N = d.N, sh = d.N * d.C, sw = d.N * d.C * d.H;  // strides of ih and iw
  for (int pos = blockIdx.x; pos < positions; pos += gridDim.x) {
    const int c = pos % C, r = pos / C, oh = r % HO, ow = r / HO;
    const float* xb = X + N * c + sh * (oh * stride) + sw * (ow * stride);
    for (int64_t n = threadIdx.x; n < N; n += blockDim.x) {
      float mx = -INFINITY;
      int32_t mi = 0;
      for (int ph = 0; ph < pool; ++ph)
        for (int pw = 0; pw < pool; ++pw) {
          const float v = xb[n + sh * ph + sw * pw];
          if (v > mx) {
            mx = v;
            mi = ph * pool + pw;
          }
        }
      Y[n + N * pos] = mx;
      idx[n + N * pos] = mi;
    }
  }
}

// maxpool_fwd_kernel for N % 4 == 0 (and 16-byte aligned tensors): a wave
// owns a window position, its lanes stride over n in float4s, so each tap
// is one 16-byte load per lane; per element the same strict-> scan in
// (ph, pw) order as the scalar kernel.
__global__ void __launch_bounds__(256) maxpool_fwd_vec_kernel(PoolDims d, const float* __restrict__ X,
                                                              float* __restrict__ Y,
                                                              int32_t* __restrict__ idx) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  const int C = (int)d.C, HO = (int)d.HO, pool = (int)d.pool, stride = (int)d.stride;
  const int positions = C * HO * (int)d.WO;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t N = d.N, N4 = d.N >> 2, sh = d.N * d.C, sw = d.N * d.C * d.H;
  for (int pos = blockIdx.x * 4 + w; pos < positions; pos += gridDim.x * 4) {
    const int c = pos % C, r = pos / C, oh = r % HO, ow = r / HO;
    const float* xb = X + N * c + sh * (oh * stride) + sw * (ow * stride);
    for (int64_t q = lane; q < N4; q += 64) {
      f32x4 mx = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
      i32x4 mi = {0, 0, 0, 0};
      for (int ph = 0; ph < pool; ++ph)
        for (int pw = 0; pw < pool; ++pw) {
          const f32x4 v = *reinterpret_cast<const f32x4*>(xb + sh * ph + sw * pw + 4 * q);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (v[e] > mx[e]) {
              mx[e] = v[e];
              mi[e] = ph * pool + pw;
            }
        }
      *reinterpret_cast<f32x4*>(Y + N * pos + 4 * q) = mx;
      *reinterpret_cast<i32x4*>(idx + N * pos + 4 * q) = mi;
    }
  }
}

// The ReLU backward fused into the pool's backward (MASK): the pool's input
// is a ReLU output, and a routed gradient is scaled by relu_mask of that
// input at the argmax -- read from the input itself (kMaskIn: y is the ReLU
// output [N, C, H, W]) or from the pool's own output (kMaskOut: y is the
// pooled [N, C, HO, WO], whose value at a window is the input at its argmax,
// bit for bit, so the scale is the same; the ReLU output itself then need
// not be kept).
constexpr int kMaskNone = 0, kMaskIn = 1, kMaskOut = 2;

// maxpool_bwd_tiled_kernel for N % 4 == 0: a wave per window, float4s over n.
template <int MASK>
__global__ void __launch_bounds__(256) maxpool_bwd_tiled_vec_kernel(PoolDims d,
                                                                    const float* __restrict__ dY,
                                                                    const int32_t* __restrict__ idx,
                                                                    const float* __restrict__ y,
                                                                    float* __restrict__ dX) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  const int C = (int)d.C, HO = (int)d.HO, pool = (int)d.pool;
  const int positions = C * HO * (int)d.WO;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t N = d.N, N4 = d.N >> 2, sh = d.N * d.C, sw = d.N * d.C * d.H;
  for (int pos = blockIdx.x * 4 + w; pos < positions; pos += gridDim.x * 4) {
    const int c = pos % C, r = pos / C, oh = r % HO, ow = r / HO;
    const int64_t base = N * c + sh * (oh * pool) + sw * (ow * pool);
    for (int64_t q = lane; q < N4; q += 64) {
      const i32x4 mi = *reinterpret_cast<const i32x4*>(idx + N * pos + 4 * q);
      f32x4 gy = 0.f + *reinterpret_cast<const f32x4*>(dY + N * pos + 4 * q);
      if (MASK == kMaskOut) {
        const f32x4 yv = *reinterpret_cast<const f32x4*>(y + N * pos + 4 * q);
#pragma unroll
        for (int e = 0; e < 4; ++e) gy[e] *= relu_mask(yv[e]);
      }
      for (int ph = 0; ph < pool; ++ph)
        for (int pw = 0; pw < pool; ++pw) {
          const int64_t o = base + sh * ph + sw * pw + 4 * q;
          f32x4 g;
#pragma unroll
          for (int e = 0; e < 4; ++e) g[e] = mi[e] == ph * pool + pw ? gy[e] : 0.f;
          if (MASK == kMaskIn) {
            const f32x4 yv = *reinterpret_cast<const f32x4*>(y + o);
#pragma unroll
            for (int e = 0; e < 4; ++e) g[e] *= relu_mask(yv[e]);
          }
          *reinterpret_cast<f32x4*>(dX + o) = g;
        }
    }
  }
}

// Backward as a gather (any stride): input position (c, ih, iw) sums dY over
// the windows that contain it and picked it, in (oh, ow) order starting from
// 0, then scales by the ReLU mask (kMaskIn), or scales each window's term
// (kMaskOut; the same value wherever the mask is 1).
template <int MASK>
__global__ void __launch_bounds__(256) maxpool_bwd_gather_kernel(PoolDims d,
                                                                 const float* __restrict__ dY,
                                                                 const int32_t* __restrict__ idx,
                                                                 const float* __restrict__ y,
                                                                 float* __restrict__ dX) {
  const int C = (int)d.C, H = (int)d.H, HO = (int)d.HO, WO = (int)d.WO;
  const int pool = (int)d.pool, stride = (int)d.stride;
  const int positions = C * H * (int)d.W;
  const int64_t N = d.N;
  for (int pos = blockIdx.x; pos < positions; pos += gridDim.x) {
    const int c = pos % C, r = pos / C, ih = r % H, iw = r / H;
    // windows (oh, ow) with oh*stride <= ih < oh*stride + pool
    const int oh_lo = ih >= pool ? (ih - pool) / stride + 1 : 0;
    const int oh_hi = min(ih / stride, HO - 1);
    const int ow_lo = iw >= pool ? (iw - pool) / stride + 1 : 0;
    const int ow_hi = min(iw / stride, WO - 1);
    for (int64_t n = threadIdx.x; n < N; n += blockDim.x) {
      float g = 0.f;
      for (int oh = oh_lo; oh <= oh_hi; ++oh)
        for (int ow = ow_lo; ow <= ow_hi; ++ow) {
          const int32_t want = (ih - oh * stride) * pool + (iw - ow * stride);
          const int64_t o = n + N * (c + (int64_t)C * (oh + HO * ow));
          if (idx[o] == want) g += MASK == kMaskOut ? dY[o] * relu_mask(y[o]) : dY[o];
        }
      if (MASK == kMaskIn) g *= relu_mask(y[n + N * pos]);
      dX[n + N * pos] = g;
    }
  }
}

// Backward when the windows tile the input exactly (stride == pool, H and W
// multiples of pool): each input element lies in exactly one window, so a
// block per window reads idx/dY once and writes its pool^2 inputs:
// 0 + dY at the argmax (the reference's zero-fill then add), 0 elsewhere.
template <int MASK>
__global__ void __launch_bounds__(256) maxpool_bwd_tiled_kernel(PoolDims d,
                                                                const float* __restrict__ dY,
                                                                const int32_t* __restrict__ idx,
                                                                const float* __restrict__ y,
                                                                float* __restrict__ dX) {
  const int C = (int)d.C, HO = (int)d.HO, pool = (int)d.pool;
  const int positions = C * HO * (int)d.WO;
  const int64_t N = d.N, sh = d.N * d.C, sw = d.N * d.C * d.H;
  for (int pos = blockIdx.x; pos < positions; pos += gridDim.x) {
    const int c = pos % C, r = pos / C, oh = r % HO, ow = r / HO;
    const int64_t base = N * c + sh * (oh * pool) + sw * (ow * pool);
    for (int64_t n = threadIdx.x; n < N; n += blockDim.x) {
      const int32_t mi = idx[n + N * pos];
      float gy = 0.f + dY[n + N * pos];
      if (MASK == kMaskOut) gy *= relu_mask(y[n + N * pos]);
      for (int ph = 0; ph < pool; ++ph)
        for (int pw = 0; pw < pool; ++pw) {
          const int64_t o = base + n + sh * ph + sw * pw;
          float g = mi == ph * pool + pw ? gy : 0.f;
          if (MASK == kMaskIn) g *= relu_mask(y[o]);
          dX[o] = g;
        }
    }
  }
}

// Backward of a classifier head Conv2D -> ReLU -> MaxPool2D -> Flatten ->
// Linear(F -> O) from the Linear's output gradient dZ [N, O] down to the
// ReLU's input, in one pass over the pooled output P [N, F] (the Linear's
// input, F = C HO WO, f = c + C (oh + HO ow)):
//   gW[f, o] (+)= sum_n P[n, f] dZ[n, o]      gb[o] (+)= sum_n dZ[n, o]
//   dX = the pool's routing of (dZ W^T)[n, f] * [P[n, f] > 0]
// A wave takes a feature f: lane l runs over n = l, l + 64, ... in order and
// the lane sums meet in an xor butterfly -- the order gemm_small_wave_kernel
// sums a weight gradient in (and its bias column sums), so gW and gb are bit
// for bit the separate Linear backward's where that kernel serves it (the
// float4 form below, for N % 4 == 0, sums each lane's 4 rows first).  The
// input gradient (dZ W^T)[n, f] is summed over o ascending, then masked and
// routed as maxpool_bwd_tiled_vec_kernel<kMaskOut> does.  dZ is staged in LDS
// per block; each P and argmax element is read once, each dX element written
// once (the windows tile the input).
constexpr int kLinPoolMaxO = 16, kLinPoolMaxNO = 8192;

// O (outputs) and POOL (window, 0 = taken from d) are compile-time, so the
// per-row loops unroll without guards and their LDS reads issue together.
template <int O, int POOL>
__global__ void __launch_bounds__(256) linear_bwd_maxpool_kernel(PoolDims d, const float* __restrict__ P,
                                                                 const int32_t* __restrict__ idx,
                                                                 const float* __restrict__ W,
                                                                 const float* __restrict__ dZ, float* __restrict__ gW,
                                                                 float* __restrict__ gb, float* __restrict__ dX,
                                                                 int accumulate) {
  __shared__ float dzs[kLinPoolMaxNO];
  const int N = (int)d.N, C = (int)d.C, HO = (int)d.HO;
  const int pool = POOL > 0 ? POOL : (int)d.pool;
  const int F = C * HO * (int)d.WO;
  {
    // 16 loads in flight per thread before their LDS stores: one round trip
    // for up to 4096 floats of dZ
    constexpr int U = 16;
    const int NO = N * O;
    for (int e0 = 0; e0 < NO; e0 += 256 * U) {
      float v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int e = e0 + (int)threadIdx.x + 256 * u;
        v[u] = e < NO ? dZ[e] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int e = e0 + (int)threadIdx.x + 256 * u;
        if (e < NO) dzs[e] = v[u];
      }
    }
  }
  __syncthreads();
  // the wave index as a wave-uniform value: a feature's W row then comes
  // through scalar loads
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t sh = d.N * d.C, sw = d.N * d.C * d.H;
  const int fstride = gridDim.x * 4;
  for (int f = blockIdx.x * 4 + w; f < F; f += fstride) {
    const int c = f % C, r = f / C, oh = r % HO, ow = r / HO;
    const int64_t base = d.N * c + sh * (oh * pool) + sw * (ow * pool);
    const float* pf = P + d.N * f;
    const int32_t* xf = idx + d.N * f;
    float wf[O], acc[O];
#pragma unroll
    for (int o = 0; o < O; ++o) {
      wf[o] = W[f + (int64_t)F * o];
      acc[o] = 0.f;
    }
    for (int n0 = 0; n0 < N; n0 += 256) {
      // the lane's four rows loaded together, then all four computed, then
      // all their stores: a store ahead of a load would make the wait for
      // that load wait for the store as well (vmcnt counts both)
      float x[4], g[4];
      int mi[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int n = n0 + lane + 64 * u;
        x[u] = n < N ? pf[n] : 0.f;
        mi[u] = n < N ? xf[n] : -1;
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int n = n0 + lane + 64 * u;
        const bool ok = n < N;
        const int nr = ok ? n : N - 1;
        float dz[O];
#pragma unroll
        for (int o = 0; o < O; ++o) dz[o] = dzs[nr + N * o];
        float gv = 0.f;
#pragma unroll
        for (int o = 0; o < O; ++o) {
          const float a = fmaf(x[u], dz[o], acc[o]);
          acc[o] = ok ? a : acc[o];
          gv = fmaf(dz[o], wf[o], gv);
        }
        g[u] = (0.f + gv) * relu_mask(x[u]);
      }
      auto store = [&](int u) {
        const int n = n0 + lane + 64 * u;
        if (POOL > 0) {
#pragma unroll
          for (int ph = 0; ph < (POOL > 0 ? POOL : 1); ++ph)
#pragma unroll
            for (int pw = 0; pw < (POOL > 0 ? POOL : 1); ++pw)
              dX[base + n + sh * ph + sw * pw] = mi[u] == ph * pool + pw ? g[u] : 0.f;
        } else {
          for (int ph = 0; ph < pool; ++ph)
            for (int pw = 0; pw < pool; ++pw)
              dX[base + n + sh * ph + sw * pw] = mi[u] == ph * pool + pw ? g[u] : 0.f;
        }
      };
      if (n0 + 256 <= N) {  // wave-uniform: a full set of rows, no per-row branch
#pragma unroll
        for (int u = 0; u < 4; ++u) store(u);
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (n0 + lane + 64 * u < N) store(u);
      }
    }
#pragma unroll
    for (int o = 0; o < O; ++o) {
      float a = acc[o];
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) a += __shfl_xor(a, off, 64);
      acc[o] = a;
    }
    if (lane == 0) {
      float prev[O];
#pragma unroll
      for (int o = 0; o < O; ++o) prev[o] = accumulate ? gW[f + (int64_t)F * o] : 0.f;
#pragma unroll
      for (int o = 0; o < O; ++o) gW[f + (int64_t)F * o] = accumulate ? acc[o] + prev[o] : acc[o];
    }
  }
  // bias gradient: output o = 4 block + wave sums dZ's column o, after the
  // features (one column per wave, so no wave's features wait for it)
  const int o = blockIdx.x * 4 + w;
  if (gb && o < O) {
    float sum = 0.f;
    for (int n = lane; n < N; n += 64) sum += dzs[n + N * o];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
    if (lane == 0) gb[o] = accumulate ? gb[o] + sum : sum;
  }
}

// linear_bwd_maxpool_kernel for N % 4 == 0 with 16-byte accesses: lane l
// owns rows 4 l .. 4 l + 3 (+ 256 j), so P, the argmax and dZ's LDS rows come
// as float4 / int4 and dX leaves as float4s.  A lane sums its rows in
// ascending order, then the lanes meet in the xor butterfly (a fixed order;
// not the separate weight-gradient kernel's lane-strided one).
template <int O, int POOL>
__global__ void __launch_bounds__(256) linear_bwd_maxpool_vec_kernel(PoolDims d, const float* __restrict__ P,
                                                                     const int32_t* __restrict__ idx,
                                                                     const float* __restrict__ W,
                                                                     const float* __restrict__ dZ,
                                                                     float* __restrict__ gW, float* __restrict__ gb,
                                                                     float* __restrict__ dX, int accumulate) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  __shared__ __align__(16) float dzs[kLinPoolMaxNO];
  const int N = (int)d.N, C = (int)d.C, HO = (int)d.HO;
  const int pool = POOL > 0 ? POOL : (int)d.pool;
  const int F = C * HO * (int)d.WO;
  {
    constexpr int U = 4;  // float4s in flight per thread: 4096 floats of dZ per round trip
    const int NO4 = N * O / 4;
    for (int e0 = 0; e0 < NO4; e0 += 256 * U) {
      f32x4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int e = e0 + (int)threadIdx.x + 256 * u;
        v[u] = e < NO4 ? reinterpret_cast<const f32x4*>(dZ)[e] : f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int e = e0 + (int)threadIdx.x + 256 * u;
        if (e < NO4) reinterpret_cast<f32x4*>(dzs)[e] = v[u];
      }
    }
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t sh = d.N * d.C, sw = d.N * d.C * d.H;
  for (int f = blockIdx.x * 4 + w; f < F; f += gridDim.x * 4) {
    const int c = f % C, r = f / C, oh = r % HO, ow = r / HO;
    const int64_t base = d.N * c + sh * (oh * pool) + sw * (ow * pool);
    const f32x4* pf = reinterpret_cast<const f32x4*>(P + d.N * f);
    const i32x4* xf = reinterpret_cast<const i32x4*>(idx + d.N * f);
    float wf[O], acc[O];
#pragma unroll
    for (int o = 0; o < O; ++o) {
      wf[o] = W[f + (int64_t)F * o];
      acc[o] = 0.f;
    }
    for (int n0 = 0; n0 < N; n0 += 256) {
      const int q = n0 / 4 + lane;  // float4 index of rows 4 q .. 4 q + 3
      if (4 * q < N) {
        const f32x4 x = pf[q];
        const i32x4 mi = xf[q];
        f32x4 g = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int o = 0; o < O; ++o) {
          const f32x4 dz = reinterpret_cast<const f32x4*>(dzs + N * o)[q];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            acc[o] = fmaf(x[e], dz[e], acc[o]);
            g[e] = fmaf(dz[e], wf[o], g[e]);
          }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) g[e] = (0.f + g[e]) * relu_mask(x[e]);
        f32x4* out = reinterpret_cast<f32x4*>(dX + base) + q;
        if (POOL > 0) {
#pragma unroll
          for (int ph = 0; ph < (POOL > 0 ? POOL : 1); ++ph)
#pragma unroll
            for (int pw = 0; pw < (POOL > 0 ? POOL : 1); ++pw) {
              f32x4 v;
#pragma unroll
              for (int e = 0; e < 4; ++e) v[e] = mi[e] == ph * pool + pw ? g[e] : 0.f;
              out[(sh * ph + sw * pw) / 4] = v;
            }
        } else {
          for (int ph = 0; ph < pool; ++ph)
            for (int pw = 0; pw < pool; ++pw) {
              f32x4 v;
#pragma unroll
              for (int e = 0; e < 4; ++e) v[e] = mi[e] == ph * pool + pw ? g[e] : 0.f;
              out[(sh * ph + sw * pw) / 4] = v;
            }
        }
      }
    }
#pragma unroll
    for (int o = 0; o < O; ++o) {
      float a = acc[o];
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) a += __shfl_xor(a, off, 64);
      acc[o] = a;
    }
    if (lane == 0) {
      float prev[O];
#pragma unroll
      for (int o = 0; o < O; ++o) prev[o] = accumulate ? gW[f + (int64_t)F * o] : 0.f;
#pragma unroll
      for (int o = 0; o < O; ++o) gW[f + (int64_t)F * o] = accumulate ? acc[o] + prev[o] : acc[o];
    }
  }
  // bias gradient: output o = 4 block + wave sums dZ's column o (each lane
  // its four rows in order, then the butterfly)
  const int o = blockIdx.x * 4 + w;
  if (gb && o < O) {
    float sum = 0.f;
    for (int q = lane; 4 * q < N; q += 64) {
      const f32x4 dz = reinterpret_cast<const f32x4*>(dzs + N * o)[q];
      sum += dz[0];
      sum += dz[1];
      sum += dz[2];
      sum += dz[3];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
    if (lane == 0) gb[o] = accumulate ? gb[o] + sum : sum;
  }
}

template <int O>
void launch_linear_bwd_maxpool(unsigned grid, hipStream_t st, const PoolDims& d, const float* P,
                               const int32_t* idx, const float* W, const float* dZ, float* gW, float* gb,
                               float* dX, int accumulate) {
  const bool vec = d.N % 4 == 0 && aligned16(P) && aligned16(idx) && aligned16(dZ) && aligned16(dX);
  if (vec && d.pool == 2)
    hipLaunchKernelGGL((linear_bwd_maxpool_vec_kernel<O, 2>), dim3(grid), dim3(256), 0, st, d, P, idx, W, dZ, gW,
                       gb, dX, accumulate);
  else if (vec)
    hipLaunchKernelGGL((linear_bwd_maxpool_vec_kernel<O, 0>), dim3(grid), dim3(256), 0, st, d, P, idx, W, dZ, gW,
                       gb, dX, accumulate);
  else if (d.pool == 2)
    hipLaunchKernelGGL((linear_bwd_maxpool_kernel<O, 2>), dim3(grid), dim3(256), 0, st, d, P, idx, W, dZ, gW, gb,
                       dX, accumulate);
  else
    hipLaunchKernelGGL((linear_bwd_maxpool_kernel<O, 0>), dim3(grid), dim3(256), 0, st, d, P, idx, W, dZ, gW, gb,
                       dX, accumulate);
}

template <int... Os>
void dispatch_linear_bwd_maxpool(std::integer_sequence<int, Os...>, int O, unsigned grid, hipStream_t st,
                                 const PoolDims& d, const float* P, const int32_t* idx, const float* W,
                                 const float* dZ, float* gW, float* gb, float* dX, int accumulate) {
  ((O == Os + 1 ? launch_linear_bwd_maxpool<Os + 1>(grid, st, d, P, idx, W, dZ, gW, gb, dX, accumulate) : void()),
   ...);
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

unsigned pool_grid(int64_t positions) {
  return (unsigned)(positions < kPoolGrid ? positions : kPoolGrid);
}
unsigned pool_threads(int64_t N) { return N >= 256 ? 256u : (unsigned)((N + 63) / 64 * 64); }

// y: null, the pool's input (a ReLU output; mask kMaskIn) or the pool's
// output (mask kMaskOut), see maxpool_bwd_tiled_vec_kernel.
int maxpool_backward(const float* dY, const int32_t* idx, const float* y, int mask, float* dX, int64_t N,
                     int64_t C, int64_t H, int64_t W, int64_t pool, int64_t stride,
                     cnhip_stream_t stream, const char* who) {
  PoolDims d;
  CNHIP_TRY(pool_dims(d, N, C, H, W, pool, stride, who));
  CNHIP_REQUIRE(dY && idx && dX, "%s: NULL pointer", who);
  CNHIP_REQUIRE(C * H * W < ((int64_t)1 << 31), "%s: too many input positions", who);
  const hipStream_t st = as_stream(stream);
  const unsigned threads = pool_threads(N);
  // dY and the argmax read per output; dX written per input; the mask's
  // source read per input (kMaskIn) or per output (kMaskOut)
  if (!y) mask = kMaskNone;
  const double outs = (double)N * C * d.HO * d.WO, ins = (double)N * C * H * W;
  const double bytes = 8.0 * outs + 4.0 * ins + (mask == kMaskIn ? 4.0 * ins : mask == kMaskOut ? 4.0 * outs : 0.0);
  HbmTimer timer(mask == kMaskIn ? "maxpool_bwd_kernel<relu>"
                 : mask == kMaskOut ? "maxpool_bwd_kernel<relu of output>"
                                    : "maxpool_bwd_kernel",
                 bytes, st);
  const bool vec = N % 4 == 0 && aligned16(dY) && aligned16(idx) && aligned16(dX) && (!y || aligned16(y));
  const bool tiled = d.stride == d.pool && d.HO * d.pool == H && d.WO * d.pool == W;
  auto go = [&](auto mode) {
    constexpr int M = decltype(mode)::value;
    if (tiled && vec) {
      const unsigned grid = pool_grid((C * d.HO * d.WO + 3) / 4);
      hipLaunchKernelGGL(maxpool_bwd_tiled_vec_kernel<M>, dim3(grid), dim3(256), 0, st, d, dY, idx, y, dX);
    } else if (tiled) {
      hipLaunchKernelGGL(maxpool_bwd_tiled_kernel<M>, dim3(pool_grid(C * d.HO * d.WO)), dim3(threads), 0, st, d,
                         dY, idx, y, dX);
    } else {
      hipLaunchKernelGGL(maxpool_bwd_gather_kernel<M>, dim3(pool_grid(C * H * W)), dim3(threads), 0, st, d, dY,
                         idx, y, dX);
    }
  };
  if (mask == kMaskIn)
    go(std::integral_constant<int, kMaskIn>{});
  else if (mask == kMaskOut)
    go(std::integral_constant<int, kMaskOut>{});
  else
    go(std::integral_constant<int, kMaskNone>{});
  return check_launch(who);
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
  const int64_t positions = C * d.HO * d.WO;
  CNHIP_REQUIRE(positions < ((int64_t)1 << 31), "%s: too many output positions", who);
  // X read once; Y and the int32 argmax written
  cnhip::HbmTimer timer("maxpool_fwd_kernel", 4.0 * (double)N * C * H * W + 8.0 * (double)N * positions,
                        cnhip::as_stream(stream));
  if (N % 4 == 0 && cnhip::aligned16(X) && cnhip::aligned16(Y) && cnhip::aligned16(idx))
    hipLaunchKernelGGL(cnhip::maxpool_fwd_vec_kernel, dim3(cnhip::pool_grid((positions + 3) / 4)), dim3(256),
                       0, cnhip::as_stream(stream), d, X, Y, idx);
  else
    hipLaunchKernelGGL(cnhip::maxpool_fwd_kernel, dim3(cnhip::pool_grid(positions)),
                       dim3(cnhip::pool_threads(N)), 0, cnhip::as_stream(stream), d, X, Y, idx);
  return cnhip::check_launch(who);
}

int cnhip_maxpool2d_backward(const float* dY, const int32_t* idx, float* dX, int64_t N, int64_t C,
                             int64_t H, int64_t W, int64_t pool, int64_t stride,
                             cnhip_stream_t stream) {
  return cnhip::maxpool_backward(dY, idx, nullptr, cnhip::kMaskNone, dX, N, C, H, W, pool, stride, stream,
                                 "cnhip_maxpool2d_backward");
}

int cnhip_maxpool2d_backward_relu(const float* dY, const int32_t* idx, const float* y, float* dX,
                                  int64_t N, int64_t C, int64_t H, int64_t W, int64_t pool,
                                  int64_t stride, cnhip_stream_t stream) {
  const char* who = "cnhip_maxpool2d_backward_relu";
  CNHIP_REQUIRE(y, "%s: NULL ReLU output", who);
  return cnhip::maxpool_backward(dY, idx, y, cnhip::kMaskIn, dX, N, C, H, W, pool, stride, stream, who);
}

int cnhip_maxpool2d_backward_relu_pooled(const float* dY, const int32_t* idx, const float* Y, float* dX,
                                         int64_t N, int64_t C, int64_t H, int64_t W, int64_t pool,
                                         int64_t stride, cnhip_stream_t stream) {
  const char* who = "cnhip_maxpool2d_backward_relu_pooled";
  CNHIP_REQUIRE(Y, "%s: NULL pooled output", who);
  return cnhip::maxpool_backward(dY, idx, Y, cnhip::kMaskOut, dX, N, C, H, W, pool, stride, stream, who);
}

int cnhip_linear_backward_maxpool_relu_fits(int64_t N, int64_t C, int64_t H, int64_t W, int64_t out_features,
                                            int64_t pool, int64_t stride) {
  if (stride <= 0) stride = pool;
  return N > 0 && C > 0 && pool > 0 && stride == pool && H % pool == 0 && W % pool == 0 && out_features > 0 &&
                 out_features <= cnhip::kLinPoolMaxO && N * out_features <= cnhip::kLinPoolMaxNO &&
                 C * H * W < ((int64_t)1 << 31)
             ? 1
             : 0;
}

int cnhip_linear_backward_maxpool_relu(const float* P, const int32_t* idx, const float* W, const float* dZ,
                                       float* grad_W, float* grad_b, float* dX, int64_t N, int64_t C, int64_t H,
                                       int64_t Wd, int64_t out_features, int64_t pool, int64_t stride, int accumulate,
                                       cnhip_stream_t stream) {
  const char* who = "cnhip_linear_backward_maxpool_relu";
  cnhip::PoolDims d;
  CNHIP_TRY(cnhip::pool_dims(d, N, C, H, Wd, pool, stride, who));
  CNHIP_REQUIRE(cnhip_linear_backward_maxpool_relu_fits(N, C, H, Wd, out_features, pool, stride),
                "%s: needs windows that tile the input (stride == pool dividing H and W), out_features <= %d and "
                "batch * out_features <= %d (N=%lld C=%lld H=%lld W=%lld out=%lld pool=%lld stride=%lld)",
                who, cnhip::kLinPoolMaxO, cnhip::kLinPoolMaxNO, (long long)N, (long long)C, (long long)H,
                (long long)Wd, (long long)out_features, (long long)pool, (long long)stride);
  CNHIP_REQUIRE(P && idx && W && dZ && grad_W && dX, "%s: NULL pointer", who);
  const hipStream_t st = cnhip::as_stream(stream);
  const int64_t F = C * d.HO * d.WO;
  // P and the argmax read once, dX written once, grad_W written (and read
  // when accumulating); dZ and W are small
  const double bytes = 8.0 * (double)N * F + 4.0 * (double)N * C * H * Wd +
                       (accumulate ? 8.0 : 4.0) * (double)F * out_features + 4.0 * (double)N * out_features;
  cnhip::HbmTimer timer("linear_bwd_maxpool_kernel", bytes, st);
  // a wave per feature (up to 1024 blocks), and at least one wave per output
  // for the bias gradient
  const unsigned grid = (unsigned)std::max<int64_t>(std::min<int64_t>((F + 3) / 4, 1024), (out_features + 3) / 4);
  cnhip::dispatch_linear_bwd_maxpool(std::make_integer_sequence<int, cnhip::kLinPoolMaxO>{}, (int)out_features,
                                     grid, st, d, P, idx, W, dZ, grad_W, grad_b, dX, accumulate);
  return cnhip::check_launch(who);
}

}  // extern "C"
