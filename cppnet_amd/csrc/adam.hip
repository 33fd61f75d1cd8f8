// Fused single-pass Adam: one read of W, g, m, v and one write of W, m, v
// per parameter (28 bytes), float4-vectorised, over one or many tensors in a
// single launch.
//
// ref: adam_step.cu:10-25 and Adam::update, src/CppNet/optimizers/adam.cpp:98-133.
// The update is evaluated with the same sequence of fp32 roundings as the
// reference host loop (no fused multiply-add contraction), so it is
// bit-identical to it for identical inputs:
//   m = b1*m + (1-b1)*g ; v = b2*v + (1-b2)*g*g ; mh = m/bc1 ; vh = v/bc2
//   W -= lr*mh / (sqrt(vh) + eps)
#include <hip/hip_runtime.h>

#include "common.hpp"
#include "optim_math.hpp"

namespace cnhip {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int MAX_TENSORS = 64;
constexpr int ADAM_BLOCK = 256;


struct AdamTensor {
  float* W;
  const float* g;
  float* m;
  float* v;
  int64_t n;
  float bc1, bc2;
  int vec;
  int first_block;  // prefix sum of blocks over the tensors before this one
};

struct AdamBatch {
  AdamTensor t[MAX_TENSORS];
  int count;
};

// A block updates R * ADAM_BLOCK * 4 consecutive values of one tensor.  In
// the float4 path every thread first loads all R of its float4s of W, g, m
// and v (4R loads in flight), then updates them, then stores: the four
// arrays are distinct buffers, so no store can feed a later load.
template <int R>
__device__ __forceinline__ void adam_range(const AdamTensor& T, int64_t begin, const AdamHyper& h,
                                           const UpdateGuard& guard) {
  if (T.vec) {
    // begin is a multiple of the chunk, hence of 4.
    f32x4 w[R], g[R], m[R], v[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t i = begin + ((int64_t)r * ADAM_BLOCK + threadIdx.x) * 4;
      if (i < T.n) {
        w[r] = *reinterpret_cast<const f32x4*>(T.W + i);
        g[r] = *reinterpret_cast<const f32x4*>(T.g + i);
        m[r] = *reinterpret_cast<const f32x4*>(T.m + i);
        v[r] = *reinterpret_cast<const f32x4*>(T.v + i);
      }
    }
    if (update_withheld(guard)) return;  // checked once the loads are in flight
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float we = w[r][e], me = m[r][e], ve = v[r][e];
        adam_one(we, g[r][e], me, ve, T.bc1, T.bc2, h);
        w[r][e] = we; m[r][e] = me; v[r][e] = ve;
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t i = begin + ((int64_t)r * ADAM_BLOCK + threadIdx.x) * 4;
      if (i < T.n) {
        *reinterpret_cast<f32x4*>(T.W + i) = w[r];
        *reinterpret_cast<f32x4*>(T.m + i) = m[r];
        *reinterpret_cast<f32x4*>(T.v + i) = v[r];
      }
    }
  } else {
    if (update_withheld(guard)) return;
    for (int r = 0; r < 4 * R; ++r) {
      const int64_t i = begin + (int64_t)r * ADAM_BLOCK + threadIdx.x;
      if (i >= T.n) break;
      float w = T.W[i], m = T.m[i], v = T.v[i];
      adam_one(w, T.g[i], m, v, T.bc1, T.bc2, h);
      T.W[i] = w; T.m[i] = m; T.v[i] = v;
    }
  }
}

template <int R>
__global__ void __launch_bounds__(ADAM_BLOCK) adam_multi_kernel(AdamBatch batch, AdamHyper h, UpdateGuard guard) {
  // Find the tensor owning this block (count <= 64: a linear scan of
  // uniform values is cheap and stays in scalar registers).
  int ti = 0;
  for (int i = 1; i < batch.count; ++i)
    if ((int)blockIdx.x >= batch.t[i].first_block) ti = i;
  const AdamTensor& T = batch.t[ti];
  const int64_t begin = (int64_t)((int)blockIdx.x - T.first_block) * (R * ADAM_BLOCK * 4);
  adam_range<R>(T, begin, h, guard);
}

template <int R>
int adam_launch_r(AdamBatch& b, const AdamHyper& h, int64_t params, hipStream_t st, const char* who) {
  constexpr int64_t chunk = R * ADAM_BLOCK * 4;
  int blocks = 0;
  for (int i = 0; i < b.count; ++i) {
    b.t[i].first_block = blocks;
    const int64_t nb = (b.t[i].n + chunk - 1) / chunk;
    CNHIP_REQUIRE(blocks + nb < (int64_t)1 << 30, "%s: too many parameters", who);
    blocks += (int)nb;
  }
  if (blocks == 0) return CNHIP_OK;
  UpdateGuard guard;
  CNHIP_TRY(update_guard(&guard, who));
  // read W, g, m, v and write W, m, v: 28 bytes per parameter
  HbmTimer timer("adam_multi_kernel", 28.0 * (double)params, st);
  hipLaunchKernelGGL(adam_multi_kernel<R>, dim3(blocks), dim3(ADAM_BLOCK), 0, st, b, h, guard);
  return check_launch(who);
}

// Four float4s per thread for large updates; fewer when that would leave
// the 256 CUs with fewer than ~8 blocks each.
int adam_launch(AdamBatch& b, const AdamHyper& h, hipStream_t st, const char* who) {
  int64_t params = 0;
  for (int i = 0; i < b.count; ++i) params += b.t[i].n;
  if (params >= (int64_t)2048 * 4 * ADAM_BLOCK * 4) return adam_launch_r<4>(b, h, params, st, who);
  if (params >= (int64_t)2048 * 2 * ADAM_BLOCK * 4) return adam_launch_r<2>(b, h, params, st, who);
  return adam_launch_r<1>(b, h, params, st, who);
}

int fill_tensor(AdamTensor& T, float* W, const float* g, float* m, float* v, int64_t n, float bc1,
                float bc2, const char* who) {
  CNHIP_REQUIRE(n >= 0, "%s: negative size", who);
  CNHIP_REQUIRE(n == 0 || (W && g && m && v), "%s: NULL pointer", who);
  CNHIP_REQUIRE(bc1 != 0.f && bc2 != 0.f, "%s: bias correction is zero (step t must be >= 1)", who);
  T.W = W; T.g = g; T.m = m; T.v = v; T.n = n; T.bc1 = bc1; T.bc2 = bc2;
  T.vec = (n % 4 == 0) && aligned16(W) && aligned16(g) && aligned16(m) && aligned16(v);
  T.first_block = 0;
  return CNHIP_OK;
}

}  // namespace
}  // namespace cnhip

extern "C" {

int cnhip_adam_step(float* W, const float* g, float* m, float* v, int64_t n, float lr,
                    float beta1, float beta2, float eps, float bc1, float bc2,
                    cnhip_stream_t stream) {
  const char* who = "cnhip_adam_step";
  cnhip::AdamBatch b;
  b.count = 1;
  CNHIP_TRY(cnhip::fill_tensor(b.t[0], W, g, m, v, n, bc1, bc2, who));
  cnhip::AdamHyper h{lr, beta1, beta2, eps};
  return cnhip::adam_launch(b, h, cnhip::as_stream(stream), who);
}

int cnhip_adam_step_multi(int count, float* const* W, const float* const* g, float* const* m,
                          float* const* v, const int64_t* n, const float* bc1, const float* bc2,
                          float lr, float beta1, float beta2, float eps, cnhip_stream_t stream) {
  const char* who = "cnhip_adam_step_multi";
  CNHIP_REQUIRE(count >= 0 && count <= cnhip::MAX_TENSORS, "%s: count %d outside [0, %d]", who,
                count, cnhip::MAX_TENSORS);
  if (count == 0) return CNHIP_OK;
  CNHIP_REQUIRE(W && g && m && v && n && bc1 && bc2, "%s: NULL host array", who);
  cnhip::AdamBatch b;
  b.count = count;
  for (int i = 0; i < count; ++i)
    CNHIP_TRY(cnhip::fill_tensor(b.t[i], W[i], g[i], m[i], v[i], n[i], bc1[i], bc2[i], who));
  cnhip::AdamHyper h{lr, beta1, beta2, eps};
  return cnhip::adam_launch(b, h, cnhip::as_stream(stream), who);
}

}  // extern "C"
