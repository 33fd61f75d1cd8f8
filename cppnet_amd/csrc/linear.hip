// Linear layer entry points and the bias-gradient column reduction.
//
// ref: Linear::forward_gpu / backward_gpu, src/CppNet/layers/linear.cpp:456-539
// and the cpu-eigen semantics they must match, linear.cpp:218-234, 335-358:
//   Y  = X W + b
//   dW += X^T dY      db += sum_batch dY      dX = dY W^T
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>

#include "act_math.hpp"
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

// Backward of a Linear with few outputs over a wide input (a classifier
// head, O <= 16), in one pass over X instead of the dW GEMM, its split-K
// reduce, the bias column sum and the dX GEMM:
//   dW[f, n] (+)= sum_b X[b, f] dY[b, n]      db[n] (+)= sum_b dY[b, n]
//   dX[b, f] = (sum_n dY[b, n] W[f, n]) * act'(aux[b, f])
// with act' = [aux > 0] (ReLU below), gelu'(aux) (GELU below) or 1 (none).
// X, dY, dX ColMajor with leading dimension B, W ColMajor [F, O]; the path
// takes B % SK_RB == 0 and F % SK_FBLK == 0, so no access needs a guard.
//
// A block covers SK_FBLK features and SK_RB rows; its rows' dY [SK_RB, O]
// is staged in LDS once and shared by the four waves, wave w taking features
// SK_FW w .. SK_FW (w + 1) - 1.  Lanes walk rows (coalesced: the batch is the
// contiguous dimension), SK_U row groups per iteration so SK_U * SK_FW loads
// of X are in flight, keep SK_FW x NP running sums of X * dY and write dX as
// they go.  The 64 lane sums of each dW element are then added in lane order
// through LDS into a partial [row chunk][F, O]; skinny_reduce_kernel adds the
// row chunks in order (and the chunks' db parts).  Each element of X (and
// aux) is read once and each element of dX written once.
constexpr int SK_FW = 4, SK_FBLK = 4 * SK_FW, SK_RB = 512, SK_U = 2;

template <int NP>
constexpr int sk_lds_floats() {  // dY stage, reused for the lane sums
  return SK_RB * (NP + 1) > 4 * SK_FW * NP * 64 ? SK_RB * (NP + 1) : 4 * SK_FW * NP * 64;
}

template <int NP, int ACT, bool SEP_AUX>
__global__ void __launch_bounds__(256) linear_bwd_skinny_kernel(
    const float* __restrict__ X, const float* __restrict__ W, const float* __restrict__ dY,
    const float* __restrict__ aux, float* __restrict__ partial, float* __restrict__ dX, int64_t B,
    int64_t F) {
  constexpr int O = NP;
  __shared__ __align__(16) float lds[sk_lds_floats<NP>()];
  __shared__ float w[SK_FBLK][NP];
  float* dys = lds;  // [row][n], odd row stride: no bank conflicts
  // blockIdx.x is the row chunk: consecutive blocks read consecutive 2 KB
  // pieces of the same columns, so the blocks in flight at any time cover
  // whole contiguous runs of X rather than one piece of every column
  const int64_t f0 = (int64_t)blockIdx.y * SK_FBLK;
  const int64_t r0 = (int64_t)blockIdx.x * SK_RB;
  {
    // all of a thread's loads issued before its LDS stores (a load-store
    // loop would wait for each load in turn)
    constexpr int kPer = SK_RB * O / 256;
    float v[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = threadIdx.x + 256 * j;
      v[j] = dY[r0 + i % SK_RB + B * (i / SK_RB)];
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = threadIdx.x + 256 * j;
      dys[(i % SK_RB) * (NP + 1) + i / SK_RB] = v[j];
    }
    if (threadIdx.x < SK_FBLK * NP) {
      const int fi = threadIdx.x / NP, n = threadIdx.x % NP;
      w[fi][n] = W[f0 + fi + F * n];
    }
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float* part = partial + (int64_t)blockIdx.x * (F * O + O);  // [F, O] then db[O]
  if (blockIdx.y == 0 && wave == 0) {
    // this row chunk's part of db: lane-strided sums, then a fixed butterfly
#pragma unroll
    for (int n = 0; n < O; ++n) {
      float v = 0.f;
      for (int r = lane; r < SK_RB; r += 64) v += dys[r * (NP + 1) + n];
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
      if (lane == 0) part[F * O + n] = v;
    }
  }
  const int64_t fw = f0 + SK_FW * wave;  // this wave's first feature
  float acc[SK_FW][NP];
#pragma unroll
  for (int fi = 0; fi < SK_FW; ++fi)
#pragma unroll
    for (int n = 0; n < NP; ++n) acc[fi][n] = 0.f;
  for (int r = lane; r < SK_RB; r += 64 * SK_U) {
    float x[SK_U][SK_FW], a[SK_U][SK_FW];
#pragma unroll
    for (int u = 0; u < SK_U; ++u)
#pragma unroll
      for (int fi = 0; fi < SK_FW; ++fi) {
        const int64_t i = r0 + r + 64 * u + B * (fw + fi);
        x[u][fi] = X[i];
        a[u][fi] = SEP_AUX ? aux[i] : x[u][fi];
      }
#pragma unroll
    for (int u = 0; u < SK_U; ++u) {
      const int rr = r + 64 * u;
      float dy[NP];
#pragma unroll
      for (int n = 0; n < NP; ++n) dy[n] = dys[rr * (NP + 1) + n];
#pragma unroll
      for (int fi = 0; fi < SK_FW; ++fi) {
        float v = 0.f;
#pragma unroll
        for (int n = 0; n < NP; ++n) {
          acc[fi][n] += x[u][fi] * dy[n];
          v += dy[n] * w[SK_FW * wave + fi][n];
        }
        if (dX) {
          if (ACT == 1) v *= relu_mask(a[u][fi]);
          if (ACT == 2) v *= gelu_grad_f(a[u][fi]);
          dX[r0 + rr + B * (fw + fi)] = v;
        }
      }
    }
  }
  // lane sums through LDS (the dY stage is no longer read): value e of wave
  // w at red[(w * SK_FW * NP + e) * 64 + lane], then lane e of the wave adds
  // its 64 entries in lane order
  __syncthreads();
  float* red = lds + wave * SK_FW * NP * 64;
#pragma unroll
  for (int fi = 0; fi < SK_FW; ++fi)
#pragma unroll
    for (int n = 0; n < NP; ++n) red[(fi * NP + n) * 64 + lane] = acc[fi][n];
  __syncthreads();
  if (lane < SK_FW * NP) {
    const f32x4* q = reinterpret_cast<const f32x4*>(red + lane * 64);
    float v = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const f32x4 t = q[j];
      v += t[0];
      v += t[1];
      v += t[2];
      v += t[3];
    }
    const int fi = lane / NP, n = lane % NP;
    part[fw + fi + F * n] = v;
  }
}

// out[e] (+)= sum over the row chunks, in order, of partial[chunk][e], each
// chunk's partial being [F * O] (dW) followed by [O] (db).  Loads are issued
// eight chunks at a time, then added in order.
__global__ void __launch_bounds__(256) skinny_reduce_kernel(const float* __restrict__ partial,
                                                            float* __restrict__ dW, float* __restrict__ db,
                                                            int64_t FO, int O, int chunks, int accumulate) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= FO + O || (e >= FO && !db)) return;
  const int64_t stride = FO + O;
  const float* p = partial + e;
  float v = 0.f;
  int c = 0;
  for (; c + 8 <= chunks; c += 8) {
    float q[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) q[j] = p[(int64_t)(c + j) * stride];
#pragma unroll
    for (int j = 0; j < 8; ++j) v += q[j];
  }
  for (; c < chunks; ++c) v += p[(int64_t)c * stride];
  float* o = e < FO ? dW + e : db + (e - FO);
  *o = accumulate ? *o + v : v;
}

}  // namespace

template <int NP, int ACT, bool SEP>
void skinny_launch(dim3 grid, hipStream_t st, const float* X, const float* W, const float* dY, const float* aux,
                   float* partial, float* dX, int64_t B, int64_t F) {
  hipLaunchKernelGGL((linear_bwd_skinny_kernel<NP, ACT, SEP>), grid, dim3(256), 0, st, X, W, dY, aux, partial, dX,
                     B, F);
}

template <int NP>
void skinny_launch_o(dim3 grid, hipStream_t st, int act, bool sep, const float* X, const float* W,
                     const float* dY, const float* aux, float* partial, float* dX, int64_t B, int64_t F) {
  if (act == 0) skinny_launch<NP, 0, false>(grid, st, X, W, dY, aux, partial, dX, B, F);
  else if (act == 1 && sep) skinny_launch<NP, 1, true>(grid, st, X, W, dY, aux, partial, dX, B, F);
  else if (act == 1) skinny_launch<NP, 1, false>(grid, st, X, W, dY, aux, partial, dX, B, F);
  else if (sep) skinny_launch<NP, 2, true>(grid, st, X, W, dY, aux, partial, dX, B, F);
  else skinny_launch<NP, 2, false>(grid, st, X, W, dY, aux, partial, dX, B, F);
}

// The one-pass backward above, when the shape is one it serves (O one of
// 1, 2, 4, 8, 10, 16; B % 512 == 0, F % 16 == 0, a wide input, dW wanted);
// *done says whether it ran.  CNHIP_LINEAR_ONE_PASS=0 keeps the GEMM path.
static bool skinny_serves(int64_t B, int64_t F, int64_t O, const float* X, const float* W, const float* dY,
                          const float* dW) {
  static const bool enabled = [] {
    const char* e = std::getenv("CNHIP_LINEAR_ONE_PASS");
    return !(e && e[0] == '0');
  }();
  const bool o_ok = O == 1 || O == 2 || O == 4 || O == 8 || O == 10 || O == 16;
  return enabled && o_ok && B % SK_RB == 0 && F % SK_FBLK == 0 && F / SK_FBLK <= 65535 &&
         B * F >= ((int64_t)1 << 22) && dW && X && dY && W;
}

// partials of the one-pass backward: per row chunk [F, O] then [O]
static size_t skinny_bytes(int64_t B, int64_t F, int64_t O) {
  return (size_t)((B / SK_RB) * (F * O + O)) * sizeof(float);
}

int linear_backward_skinny(const float* X, const float* W, const float* dY, float* dW, float* db,
                           float* dX, const float* aux, int64_t B, int64_t F, int64_t O,
                           int accumulate, int act, hipStream_t st, const char* who, bool* done) {
  *done = false;
  if (!skinny_serves(B, F, O, X, W, dY, dW)) return CNHIP_OK;
  CNHIP_REQUIRE(act >= 0 && act <= 2, "%s: bad activation %d", who, act);
  CNHIP_REQUIRE(act == 0 || (dX && aux), "%s: the activation derivative needs dX and its input", who);
  const int64_t chunks = B / SK_RB, FO = F * O;
  CNHIP_REQUIRE(chunks <= 0x7fffffff, "%s: too large", who);
  void* ws = nullptr;
  CNHIP_TRY(scratch(st, kScratchGemm, skinny_bytes(B, F, O), &ws, who));
  float* partial = static_cast<float*>(ws);
  *done = true;
  const bool sep = act != 0 && aux != X;
  {
    // X (and a separate aux) read once, dX written once, the partials written
    const double per = (dX ? 8.0 : 4.0) + (sep ? 4.0 : 0.0);
    HbmTimer timer("linear_bwd_skinny_kernel",
                   per * (double)B * (double)F + 4.0 * (double)B * (double)O + 4.0 * (double)(chunks * (FO + O)),
                   st);
    const dim3 grid((unsigned)chunks, (unsigned)(F / SK_FBLK));
    switch (O) {
      case 1: skinny_launch_o<1>(grid, st, act, sep, X, W, dY, aux, partial, dX, B, F); break;
      case 2: skinny_launch_o<2>(grid, st, act, sep, X, W, dY, aux, partial, dX, B, F); break;
      case 4: skinny_launch_o<4>(grid, st, act, sep, X, W, dY, aux, partial, dX, B, F); break;
      case 8: skinny_launch_o<8>(grid, st, act, sep, X, W, dY, aux, partial, dX, B, F); break;
      case 10: skinny_launch_o<10>(grid, st, act, sep, X, W, dY, aux, partial, dX, B, F); break;
      default: skinny_launch_o<16>(grid, st, act, sep, X, W, dY, aux, partial, dX, B, F); break;
    }
    CNHIP_TRY(check_launch(who));
  }
  HbmTimer timer("skinny_reduce_kernel", 4.0 * (double)(chunks * (FO + O)) + (accumulate ? 8.0 : 4.0) * (double)(FO + O),
                 st);
  hipLaunchKernelGGL(skinny_reduce_kernel, dim3((unsigned)((FO + O + 255) / 256)), dim3(256), 0, st, partial, dW, db,
                     FO, (int)O, (int)chunks, accumulate);
  return check_launch(who);
}

// Largest GEMM-slot scratch request that cnhip_linear_backward_act makes for
// these arguments (its launches run in order on one stream, so one buffer of
// this size serves them all): the one-pass partials when that path serves
// the shape, else the split-K partials of the dW GEMM; and those of the dX
// GEMM unless the one-pass kernel wrote dX (it does for every act but the
// residual sum).
size_t linear_backward_act_scratch_bytes(const float* X, const float* W, const float* dY,
                                         const float* grad_W, const float* dX, int64_t B, int64_t I,
                                         int64_t O, int trainable, int act) {
  const bool one_pass = trainable && B > 0 && skinny_serves(B, I, O, X, W, dY, grad_W);
  size_t need = one_pass ? skinny_bytes(B, I, O) : trainable ? gemm_scratch_bytes(1, 0, I, O, B, 1) : 0;
  if (dX && !(one_pass && act != CNHIP_ACT_RESIDUAL)) need = std::max(need, gemm_scratch_bytes(0, 1, B, I, O, 1));
  return need;
}

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
    bool one_pass = false;
    CNHIP_TRY(cnhip::linear_backward_skinny(X, W, dY, grad_W, grad_b, dX, nullptr, batch, in_features,
                                            out_features, accumulate, 0, st, who, &one_pass));
    if (one_pass) return CNHIP_OK;
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
  if ((act == CNHIP_ACT_RELU || act == CNHIP_ACT_GELU) && trainable && batch > 0) {
    bool one_pass = false;
    CNHIP_TRY(cnhip::linear_backward_skinny(X, W, dY, grad_W, grad_b, dX, act_aux, batch, in_features,
                                            out_features, accumulate, act == CNHIP_ACT_RELU ? 1 : 2,
                                            cnhip::as_stream(stream), who, &one_pass));
    if (one_pass) return CNHIP_OK;
  }
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
