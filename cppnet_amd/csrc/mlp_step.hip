// One training step of a two-layer perceptron with a sigmoid output, binary
// cross-entropy and Adam in two launches: the reference's quick-start binary
// classifier (README.md:102-125),
//   Linear(I, H) -> ReLU -> Linear(H, 1) -> Sigmoid, BCE, Adam  (B 512, I 30, H 64).
// Its layer-by-layer step is seven launches of a few microseconds of work
// each (two forward GEMMs, the fused sigmoid + BCE head, the input-gradient
// GEMM with the ReLU mask, two weight-gradient GEMMs with their bias sums,
// the Adam update), and the host spends longer issuing them than the GPU
// spends running them.  Here:
//   mlp2_bce_part_kernel   a block per 16 samples: the forward, the loss
//                          terms, the backward, and the block's partial sums
//                          of every gradient over its samples;
//   mlp2_bce_adam_kernel   a thread per parameter: the partials added in
//                          block order (then the loss), the gradient stored,
//                          and the Adam update.
// Per element the arithmetic is the layer-by-layer path's: the forward
// products as fma chains in k order plus the bias, the ReLU, sigmoid with
// its clamp, the BCE terms and gradient (difference over the double
// denominator, then / B), the sigmoid derivative, dz * W2 then the ReLU
// mask, and Adam's update (optim_math.hpp).  The sums over the batch (the
// weight and bias gradients, the loss) are taken in a fixed order of their
// own: over each block's 16 samples ascending, then over the blocks.
//
// ref: Linear::forward/backward (linear.cpp:146-358), ReLU (relu.cpp:97-160),
// Sigmoid (sigmoid.cpp:97-231), BinaryCrossEntropy (binary_cross_entropy.cpp:
// 143-225), Adam::update (adam.cpp:98-133).
#include <hip/hip_runtime.h>

#include "act_math.hpp"
#include "common.hpp"
#include "optim_math.hpp"

namespace cnhip {
namespace {

constexpr int kMlpRows = 16;                // samples per block of the first launch
constexpr int kMlpMaxIn = 64, kMlpMaxHid = 64;

struct Mlp2Args {
  const float* X;   // [B, I] ColMajor
  const float* Y;   // [B]
  const float* W1;  // [I, H] ColMajor
  const float* b1;  // [H]
  const float* W2;  // [H]
  const float* b2;  // [1]
  float* part;      // [B / 16][P + 1]: gW1 [I*H], gb1 [H], gW2 [H], gb2, loss
  int64_t B;
  int I, H, P;      // P = I*H + 2H + 1 parameters
  int loss_reduction, grad_reduction;
};

__device__ __forceinline__ float sigmoid_clamped(float x) {
  const float c = fmaxf(-500.f, fminf(500.f, x));
  return 1.f / (1.f + expf(-c));
}
__device__ __forceinline__ float bce_clip_p(float p) { return fmaxf(1e-7f, fminf(p, 1.0f - 1e-7f)); }

// LDS row strides: XS and AS (4 more than a row) keep float4 reads of a row
// aligned while the 16 rows start on distinct banks, for the transposing
// store of X and the head's per-sample reads of hidden outputs; a staged W1
// column gets an odd stride (ld_w1) so that a wave's 64 columns read on
// distinct banks.  Rows and columns are zero-padded to a multiple of 4 (I4,
// H4) so the k loops step by float4: the padded terms add +0 at the end of
// an fma chain.
constexpr int kXS = kMlpMaxIn + 4, kAS = kMlpMaxHid + 4, kDS = kMlpMaxHid;
// the thread mappings below: 4 waves x 4 samples in the forward, a lane per
// hidden unit, 16 x 16 tiles of 4 x 4 for the weight gradient
static_assert(kMlpRows == 16 && kMlpMaxIn == 64 && kMlpMaxHid == 64, "mlp2_bce_part_kernel's thread mappings");

__global__ void __launch_bounds__(256) mlp2_bce_part_kernel(Mlp2Args a) {
  constexpr int R = kMlpRows;
  __shared__ __align__(16) float xs[R * kXS];            // x[r][i] at r XS + i
  __shared__ float w1s[(kMlpMaxIn + 1) * kMlpMaxHid];    // W1[i][j] at i + ld_w1 j
  __shared__ __align__(16) float a1s[R * kAS];           // ReLU outputs a[r][j] at r AS + j
  __shared__ __align__(16) float da1s[R * kDS];          // dA1[r][j] at r DS + j
  __shared__ float b1s[kMlpMaxHid];
  __shared__ __align__(16) float w2s[kMlpMaxHid];
  __shared__ float dzs[R], ls[R];
  const int I = a.I, H = a.H, IH = I * H, t = threadIdx.x;
  const int I4 = (I + 3) & ~3, H4 = (H + 3) & ~3, ld_w1 = I4 + 1;
  const int64_t r0 = (int64_t)blockIdx.x * R;
  // every global load of the block issued before the first wait
  constexpr int kW = kMlpMaxIn * kMlpMaxHid / 256, kX = R * kMlpMaxIn / 256;
  float wv[kW], xv[kX];
#pragma unroll
  for (int k = 0; k < kW; ++k) {
    const int e = t + 256 * k;
    wv[k] = e < IH ? a.W1[e] : 0.f;
  }
#pragma unroll
  for (int k = 0; k < kX; ++k) {
    const int e = t + 256 * k;  // e = i R + r: 16 consecutive samples of one input
    xv[k] = e < R * I ? a.X[r0 + (e & (R - 1)) + a.B * (e / R)] : 0.f;
  }
  float bv = 0.f, w2v = 0.f;
  if (t < H) {
    bv = a.b1[t];
    w2v = a.W2[t];
  }
  const float b2 = a.b2[0];
  const float yv = t < R ? a.Y[r0 + t] : 0.f;
#pragma unroll
  for (int k = 0; k < kW; ++k) {
    const int e = t + 256 * k;
    if (e < IH) {
      const int j = e / I, i = e - j * I;
      w1s[i + ld_w1 * j] = wv[k];
    }
  }
#pragma unroll
  for (int k = 0; k < kX; ++k) {
    const int e = t + 256 * k;
    if (e < R * I) xs[(e & (R - 1)) * kXS + e / R] = xv[k];
  }
  // the zero padding: inputs I .. I4-1 of every sample and W1 rows I .. I4-1
  // of every column; units H .. H4-1 of b1 and W2 (and of a1, written below)
  if (t < 3 * R) {
    const int r = t / 3, i = I + t % 3;
    if (i < I4) xs[r * kXS + i] = 0.f;
  }
  if (t < 3 * kMlpMaxHid) {
    const int j = t / 3, i = I + t % 3;
    if (i < I4 && j < H4) w1s[i + ld_w1 * j] = 0.f;
  }
  if (t < H4) {
    b1s[t] = t < H ? bv : 0.f;
    w2s[t] = t < H ? w2v : 0.f;
  }
  __syncthreads();
  // hidden layer, a wave per 4 samples and a lane per unit:
  // z = (sum_i x_i W1[i, j] as an fma chain in i order) + b1[j], a = relu(z)
  {
    const int j = t & 63, rb = (t >> 6) * 4;
    if (j < H4) {
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
      for (int i0 = 0; i0 < I4; i0 += 4) {
        float w[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) w[q] = w1s[i0 + q + ld_w1 * j];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float4 x4 = *reinterpret_cast<const float4*>(&xs[(rb + u) * kXS + i0]);
          acc[u] = fmaf(x4.x, w[0], acc[u]);
          acc[u] = fmaf(x4.y, w[1], acc[u]);
          acc[u] = fmaf(x4.z, w[2], acc[u]);
          acc[u] = fmaf(x4.w, w[3], acc[u]);
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) a1s[(rb + u) * kAS + j] = j < H ? relu_f(acc[u] + b1s[j]) : 0.f;
    }
  }
  __syncthreads();
  // output, loss term and dz of each sample (the sigmoid + BCE head's arithmetic)
  if (t < R) {
    float acc = 0.f;
#pragma unroll 4
    for (int j0 = 0; j0 < H4; j0 += 4) {
      const float4 h4 = *reinterpret_cast<const float4*>(&a1s[t * kAS + j0]);
      const float4 w4 = *reinterpret_cast<const float4*>(&w2s[j0]);
      acc = fmaf(h4.x, w4.x, acc);
      acc = fmaf(h4.y, w4.y, acc);
      acc = fmaf(h4.z, w4.z, acc);
      acc = fmaf(h4.w, w4.w, acc);
    }
    const float p = sigmoid_clamped(acc + b2);
    const float pc = bce_clip_p(p);
    ls[t] = -(yv * logf(pc) + (1.0f - yv) * logf(1.0f - pc));
    const float diff = pc - yv;
    float gv = (float)((double)diff / ((double)pc * (1.0 - (double)pc)));
    if (a.grad_reduction == CNHIP_REDUCE_MEAN) gv /= (float)a.B;
    dzs[t] = gv * (p * (1.f - p));
  }
  __syncthreads();
  // dA1 = (dz W2^T) * relu'(a1): the input-gradient GEMM's dz * W2[j], then the mask
#pragma unroll
  for (int k = 0; k < R * kMlpMaxHid / 256; ++k) {
    const int e = t + 256 * k, r = e >> 6, j = e & 63;
    da1s[r * kDS + j] = j < H ? fmaf(dzs[r], w2s[j], 0.f) * relu_mask(a1s[r * kAS + j]) : 0.f;
  }
  __syncthreads();
  // the block's partial sums over its samples, ascending
  float* part = a.part + (int64_t)blockIdx.x * (a.P + 1);
  {
    // gW1[i, j] = sum_r x[r][i] dA1[r][j]: a 4 x 4 tile of (i, j) per thread
    const int i0 = (t & 15) * 4, j0 = (t >> 4) * 4;
    if (i0 < I && j0 < H) {
      float acc[4][4] = {};
#pragma unroll 8
      for (int r = 0; r < R; ++r) {
        const float4 x4 = *reinterpret_cast<const float4*>(&xs[r * kXS + i0]);
        const float4 d4 = *reinterpret_cast<const float4*>(&da1s[r * kDS + j0]);
        const float xr[4] = {x4.x, x4.y, x4.z, x4.w}, dr[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int q = 0; q < 4; ++q) acc[u][q] = fmaf(xr[u], dr[q], acc[u][q]);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (i0 + u < I && j0 + q < H) part[(i0 + u) + I * (j0 + q)] = acc[u][q];
    }
  }
  if (t < H) {
    float sb = 0.f, sw = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      sb += da1s[r * kDS + t];
      sw = fmaf(a1s[r * kAS + t], dzs[r], sw);
    }
    part[IH + t] = sb;
    part[IH + H + t] = sw;
  }
  if (t == 64 * 3) {  // a lane of the last wave, which has the least tile work
    float sd = 0.f, sl = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      sd += dzs[r];
      sl += ls[r];
    }
    part[a.P - 1] = sd;
    part[a.P] = sl;
  }
}

struct Mlp2Adam {
  float* W[4];
  float* G[4];
  float* M[4];
  float* V[4];
  float bc1[4], bc2[4];
  float* loss;
};

__global__ void __launch_bounds__(256) mlp2_bce_adam_kernel(Mlp2Args a, Mlp2Adam o, AdamHyper h,
                                                            UpdateGuard guard) {
  const int e = (int)(blockIdx.x * 256 + threadIdx.x);
  if (e > a.P) return;
  const int blocks = (int)(a.B / kMlpRows);
  const int IH = a.I * a.H;
  const int tsr = e < IH ? 0 : e < IH + a.H ? 1 : e < IH + 2 * a.H ? 2 : 3;
  const int off = tsr == 0 ? e : tsr == 1 ? e - IH : tsr == 2 ? e - IH - a.H : 0;
  // the parameter and its moments loaded alongside the partials
  float w = 0.f, m = 0.f, v = 0.f;
  if (e < a.P) {
    w = o.W[tsr][off];
    m = o.M[tsr][off];
    v = o.V[tsr][off];
  }
  // the partials added in block order, 32 loads in flight at a time
  constexpr int kChunk = 32;
  const float* p = a.part + e;
  const int64_t ld = a.P + 1;
  float s = 0.f;
  for (int k0 = 0; k0 < blocks; k0 += kChunk) {
    float pv[kChunk];
#pragma unroll
    for (int u = 0; u < kChunk; ++u) pv[u] = k0 + u < blocks ? p[(int64_t)(k0 + u) * ld] : 0.f;
#pragma unroll
    for (int u = 0; u < kChunk; ++u)
      if (k0 + u < blocks) s += pv[u];
  }
  if (e == a.P) {
    *o.loss = a.loss_reduction == CNHIP_REDUCE_SUM ? s : s / (float)a.B;
    return;
  }
  o.G[tsr][off] = s;
  if (update_withheld(guard)) return;
  adam_one(w, s, m, v, o.bc1[tsr], o.bc2[tsr], h);
  o.W[tsr][off] = w;
  o.M[tsr][off] = m;
  o.V[tsr][off] = v;
}

}  // namespace
}  // namespace cnhip

extern "C" int cnhip_mlp2_bce_adam_step(const float* X, const float* Y, int64_t B, int64_t I, int64_t H, float* W1,
                                        float* b1, float* W2, float* b2, float* gW1, float* gb1, float* gW2,
                                        float* gb2, float* const* m, float* const* v, const float* bc1,
                                        const float* bc2, float lr, float beta1, float beta2, float eps,
                                        int loss_reduction, int grad_reduction, float* loss,
                                        cnhip_stream_t stream) {
  const char* who = "cnhip_mlp2_bce_adam_step";
  using namespace cnhip;
  CNHIP_REQUIRE(B > 0 && B % kMlpRows == 0 && B / kMlpRows <= 65535,
                "%s: the batch (%lld) must be a positive multiple of %d", who, (long long)B, kMlpRows);
  CNHIP_REQUIRE(I >= 1 && I <= kMlpMaxIn && H >= 1 && H <= kMlpMaxHid, "%s: layer sizes %lld -> %lld (at most %d)",
                who, (long long)I, (long long)H, kMlpMaxIn);
  CNHIP_REQUIRE(X && Y && W1 && b1 && W2 && b2 && gW1 && gb1 && gW2 && gb2 && m && v && bc1 && bc2 && loss,
                "%s: NULL pointer", who);
  for (int k = 0; k < 4; ++k) {
    CNHIP_REQUIRE(m[k] && v[k], "%s: NULL Adam moment", who);
    CNHIP_REQUIRE(bc1[k] != 0.f && bc2[k] != 0.f, "%s: bias correction is zero (step t must be >= 1)", who);
  }
  CNHIP_REQUIRE((loss_reduction == CNHIP_REDUCE_MEAN || loss_reduction == CNHIP_REDUCE_SUM) &&
                    (grad_reduction == CNHIP_REDUCE_MEAN || grad_reduction == CNHIP_REDUCE_SUM),
                "%s: bad reduction", who);
  hipStream_t st = as_stream(stream);
  Mlp2Args a{X, Y, W1, b1, W2, b2, nullptr, B, (int)I, (int)H, (int)(I * H + 2 * H + 1), loss_reduction,
             grad_reduction};
  const int blocks = (int)(B / kMlpRows);
  void* ws = nullptr;
  CNHIP_TRY(scratch(st, kScratchLayer, (size_t)blocks * (size_t)(a.P + 1) * sizeof(float), &ws, who));
  a.part = static_cast<float*>(ws);
  {
    HbmTimer timer("mlp2_bce_part_kernel", 4.0 * ((double)B * (double)(I + 1) + (double)a.P) +
                                               4.0 * (double)blocks * (double)(a.P + 1), st);
    hipLaunchKernelGGL(mlp2_bce_part_kernel, dim3((unsigned)blocks), dim3(256), 0, st, a);
    CNHIP_TRY(check_launch(who));
  }
  Mlp2Adam o{};
  float* Ws[4] = {W1, b1, W2, b2};
  float* Gs[4] = {gW1, gb1, gW2, gb2};
  for (int k = 0; k < 4; ++k) {
    o.W[k] = Ws[k];
    o.G[k] = Gs[k];
    o.M[k] = m[k];
    o.V[k] = v[k];
    o.bc1[k] = bc1[k];
    o.bc2[k] = bc2[k];
  }
  o.loss = loss;
  UpdateGuard guard;
  CNHIP_TRY(update_guard(&guard, who));
  HbmTimer timer("mlp2_bce_adam_kernel", 4.0 * (double)blocks * (double)(a.P + 1) + 32.0 * (double)a.P, st);
  hipLaunchKernelGGL(mlp2_bce_adam_kernel, dim3((unsigned)((a.P + 1 + 255) / 256)), dim3(256), 0, st, a, o,
                     AdamHyper{lr, beta1, beta2, eps}, guard);
  return check_launch(who);
}
