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
#include "colsum.hpp"
#include "common.hpp"

namespace cnhip {

int linear_wgrad_small(const float* X, const float* dY, float* dW, float* db, int64_t batch,
                       int64_t in_features, int64_t out_features, int accumulate, hipStream_t st,
                       const char* who, bool* done);
int gemm_f32(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha,
             const float* A, int64_t lda, const float* B, int64_t ldb, float beta, float* C,
             int64_t ldc, const float* bias, int epilogue, hipStream_t st, const char* who);
int linear_backward_small_pair(const float* X, const float* W, const float* dY, float* dW, float* db, float* dX,
                               int64_t batch, int64_t in_features, int64_t out_features, int accumulate,
                               hipStream_t st, const char* who, bool* done);
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
  const float s = column_wave_sum(in + rows * col, rows, vec, lane);
  if (lane == 0) out[col] = accumulate ? out[col] + s : s;
}

// Backward of a Linear with few outputs over a wide input (a classifier
// head, O <= 16), in one pass over X instead of the dW GEMM, its split-K
// reduce, the bias column sum and the dX GEMM:
//   dW[f, n] (+)= sum_b X[b, f] dY[b, n]      db[n] (+)= sum_b dY[b, n]
//   dX[b, f] = (sum_n dY[b, n] W[f, n]) * act'(aux[b, f])
// with act' = [aux > 0] (ReLU below), gelu'(aux) (GELU below) or 1 (none).
// X, dY, dX ColMajor with leading dimension B, W ColMajor [F, O]; the path
// takes B % 512 == 0, F % 16 == 0 and 16-byte aligned X, dY, dX and aux,
// so every access is an aligned float4 and none needs a guard.
//
// A block covers 16 features and 256 RPL rows, one short pass: wave w owns
// features 4w .. 4w+3 of the block, a lane 4 consecutive rows in each of
// RPL 256-row groups.  Every load of the block is issued first -- the
// lane's float4s of its 4 columns of X (and of a separate aux) and of the
// NP columns of dY, per row group -- then the lane forms its 4 x NP dW sums
// (rows in order) and its dX float4s; W of the wave's features is
// wave-uniform (scalar loads).  Short blocks keep the loads of many waves
// in flight (measured on the MI355X at [4096, 4096] -> 10: 22.8 us against
// 27.2 us for 1024-row blocks that prefetch one 256-row group ahead and
// 33.1 us for lane-strided scalar loads).  The 64 lane sums of each dW
// element are added by two DPP steps within each quad of lanes (xor 1, then
// xor 2: the four lanes end equal), then the 16 quad sums in quad order
// through LDS, into a partial [row chunk][F, O] (the chunk's db from wave 0
// of the first feature block); skinny_reduce_kernel adds the row chunks in
// order.  Each element of X (and aux) is read once and each element of dX
// written once.
constexpr int SK_FW = 4, SK_FBLK = 4 * SK_FW;  // features per wave, per block
constexpr int SK_QS = 20;  // floats per value in the quad-sum area: 16 quads + pad
__host__ __device__ constexpr int sk_rpl(int np) {  // 256-row groups per block
  return np > 10 ? 1 : 2;
}

__device__ __forceinline__ float quad_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  return v;
}

template <int NP, int ACT, bool SEP_AUX>
__global__ void __launch_bounds__(256) linear_bwd_skinny_kernel(
    const float* __restrict__ X, const float* __restrict__ W, const float* __restrict__ dY,
    const float* __restrict__ aux, float* __restrict__ partial, float* __restrict__ dX, int64_t B,
    int64_t F) {
  constexpr int O = NP, FW = SK_FW, RPL = sk_rpl(NP), NV = FW * NP, NT = NV + NP;
  __shared__ __align__(16) float red[4][NT][SK_QS];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t r0 = (int64_t)blockIdx.x * (256 * RPL);
  const int64_t fw = (int64_t)blockIdx.y * SK_FBLK + FW * wave;  // this wave's first feature
  const bool with_db = blockIdx.y == 0 && wave == 0;
  const int64_t B4 = B >> 2;
  const f32x4* X4 = reinterpret_cast<const f32x4*>(X) + (r0 >> 2) + lane + B4 * fw;
  const f32x4* A4 = reinterpret_cast<const f32x4*>(SEP_AUX ? aux : X) + (r0 >> 2) + lane + B4 * fw;
  const f32x4* D4 = reinterpret_cast<const f32x4*>(dY) + (r0 >> 2) + lane;
  f32x4 x[RPL][FW], a[RPL][FW], d[RPL][NP];
#pragma unroll
  for (int g = 0; g < RPL; ++g) {
#pragma unroll
    for (int fi = 0; fi < FW; ++fi) {
      x[g][fi] = X4[64 * g + B4 * fi];
      if (SEP_AUX) a[g][fi] = A4[64 * g + B4 * fi];
    }
#pragma unroll
    for (int n = 0; n < NP; ++n) d[g][n] = D4[64 * g + B4 * n];
  }
  float wv[FW][NP];  // W[fw + fi, n], wave-uniform
#pragma unroll
  for (int fi = 0; fi < FW; ++fi)
#pragma unroll
    for (int n = 0; n < NP; ++n) wv[fi][n] = W[fw + fi + F * n];

  float acc[FW][NP], dbs[NP];
#pragma unroll
  for (int fi = 0; fi < FW; ++fi)
#pragma unroll
    for (int n = 0; n < NP; ++n) acc[fi][n] = 0.f;
#pragma unroll
  for (int n = 0; n < NP; ++n) dbs[n] = 0.f;
#pragma unroll
  for (int g = 0; g < RPL; ++g) {
    if (with_db) {
#pragma unroll
      for (int n = 0; n < NP; ++n) dbs[n] += (d[g][n][0] + d[g][n][1]) + (d[g][n][2] + d[g][n][3]);
    }
#pragma unroll
    for (int fi = 0; fi < FW; ++fi)
#pragma unroll
      for (int n = 0; n < NP; ++n) {
        acc[fi][n] += x[g][fi][0] * d[g][n][0];
        acc[fi][n] += x[g][fi][1] * d[g][n][1];
        acc[fi][n] += x[g][fi][2] * d[g][n][2];
        acc[fi][n] += x[g][fi][3] * d[g][n][3];
      }
    if (dX) {
      f32x4* dX4 = reinterpret_cast<f32x4*>(dX) + (r0 >> 2) + lane + B4 * fw;
#pragma unroll
      for (int fi = 0; fi < FW; ++fi) {
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int n = 0; n < NP; ++n) v += d[g][n] * wv[fi][n];
        const f32x4 m = SEP_AUX ? a[g][fi] : x[g][fi];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (ACT == 1) v[j] *= relu_mask(m[j]);
          if (ACT == 2) v[j] *= gelu_grad_f(m[j]);
        }
        dX4[64 * g + B4 * fi] = v;
      }
    }
  }

  // quad sums by DPP; lane m of a quad stores the values e with e % 4 == m
  // at red[wave][e][quad], then lane e of the wave adds its 16 quad sums in
  // quad order (the wave's values e >= 64 in a second pass)
  const int q = lane >> 2, m = lane & 3;
#pragma unroll
  for (int e = 0; e < NV; ++e) {
    const float s = quad_sum(acc[e / NP][e % NP]);
    if ((e & 3) == m) red[wave][e][q] = s;
  }
  if (with_db) {
#pragma unroll
    for (int n = 0; n < NP; ++n) {
      const float s = quad_sum(dbs[n]);
      if (((NV + n) & 3) == m) red[wave][NV + n][q] = s;
    }
  }
  __syncthreads();
  float* part = partial + (int64_t)blockIdx.x * (F * O + O);  // [F, O] then db[O]
  const int cnt = with_db ? NT : NV;
#pragma unroll
  for (int p = 0; p < (NT + 63) / 64; ++p) {
    const int e = lane + 64 * p;
    if (e < cnt) {
      const f32x4* r = reinterpret_cast<const f32x4*>(&red[wave][e][0]);
      float v = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x4 t = r[j];
        v += t[0];
        v += t[1];
        v += t[2];
        v += t[3];
      }
      if (e < NV) part[fw + e / NP + F * (e % NP)] = v;
      else part[F * O + (e - NV)] = v;
    }
  }
}

// Forward of a Linear with few outputs over a wide input (a classifier head,
// O <= 16):  Y[b, n] = sum_f X[b, f] W[f, n] + bias[n], in one pass over X
// instead of a split-K GEMM whose 32-wide tile would spend most of its MFMA
// work on padding.  X ColMajor with leading dimension B (16-byte aligned,
// B % 256 == 0), W ColMajor [F, O].  A block covers 256 rows (a lane's 4
// consecutive rows as one float4) and 4 fw features, wave w features fw w ..
// fw (w + 1) - 1: the lane keeps a float4 of running sums per output over
// its wave's features in ascending order (W wave-uniform: scalar loads),
// eight features' loads in flight at a time.  The four waves' sums are added
// in wave order through LDS into partial[feature chunk][B, O];
// linear_fwd_reduce_kernel adds the chunks in order and the bias.
template <int NP>
__global__ void __launch_bounds__(256) linear_fwd_skinny_kernel(const float* __restrict__ X,
                                                                const float* __restrict__ W,
                                                                float* __restrict__ partial, int64_t B,
                                                                int64_t F, int fw) {
  __shared__ __align__(16) float red[4][NP][256];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t r0 = (int64_t)blockIdx.x * 256;
  const int64_t f0 = (int64_t)blockIdx.y * 4 * fw + (int64_t)fw * wave;  // this wave's first feature
  const int64_t B4 = B >> 2;
  const f32x4* X4 = reinterpret_cast<const f32x4*>(X) + (r0 >> 2) + lane + B4 * f0;
  f32x4 acc[NP];
#pragma unroll
  for (int n = 0; n < NP; ++n) acc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int f = 0; f < fw; f += 8) {
    f32x4 x[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = X4[B4 * (f + j)];
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int n = 0; n < NP; ++n) acc[n] += x[j] * W[f0 + f + j + F * n];
  }
#pragma unroll
  for (int n = 0; n < NP; ++n) *reinterpret_cast<f32x4*>(&red[wave][n][4 * lane]) = acc[n];
  __syncthreads();
  const int t = threadIdx.x;  // row r0 + t
  float* part = partial + (int64_t)blockIdx.y * B * NP;
#pragma unroll
  for (int n = 0; n < NP; ++n) {
    float v = red[0][n][t];
    v += red[1][n][t];
    v += red[2][n][t];
    v += red[3][n][t];
    part[r0 + t + B * n] = v;
  }
}

// Y[e] = sum over the feature chunks, in order, of partial[chunk][e] (+ the
// bias of e's column); loads issued eight chunks at a time.
__global__ void __launch_bounds__(256) linear_fwd_reduce_kernel(const float* __restrict__ partial,
                                                                const float* __restrict__ bias,
                                                                float* __restrict__ Y, int64_t B, int64_t BO,
                                                                int chunks) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= BO) return;
  const float* p = partial + e;
  float v = 0.f;
  int c = 0;
  for (; c + 8 <= chunks; c += 8) {
    float q[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) q[j] = p[(int64_t)(c + j) * BO];
#pragma unroll
    for (int j = 0; j < 8; ++j) v += q[j];
  }
  for (; c < chunks; ++c) v += p[(int64_t)c * BO];
  if (bias) v += bias[e / B];
  Y[e] = v;
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
void skinny_launch_o(hipStream_t st, int act, bool sep, const float* X, const float* W, const float* dY,
                     const float* aux, float* partial, float* dX, int64_t B, int64_t F) {
  const dim3 grid((unsigned)(B / (256 * sk_rpl(NP))), (unsigned)(F / SK_FBLK));
  if (act == 0) skinny_launch<NP, 0, false>(grid, st, X, W, dY, aux, partial, dX, B, F);
  else if (act == 1 && sep) skinny_launch<NP, 1, true>(grid, st, X, W, dY, aux, partial, dX, B, F);
  else if (act == 1) skinny_launch<NP, 1, false>(grid, st, X, W, dY, aux, partial, dX, B, F);
  else if (sep) skinny_launch<NP, 2, true>(grid, st, X, W, dY, aux, partial, dX, B, F);
  else skinny_launch<NP, 2, false>(grid, st, X, W, dY, aux, partial, dX, B, F);
}

// The one-pass backward above, when the shape is one it serves (O one of
// 1, 2, 4, 8, 10, 16; B % 512 == 0, F % 16 == 0, a wide input, dW wanted,
// X, dY, dX and a separate aux 16-byte aligned); *done says whether it ran.
// CNHIP_LINEAR_ONE_PASS=0 keeps the GEMM path.
static bool skinny_serves(int64_t B, int64_t F, int64_t O, const float* X, const float* W, const float* dY,
                          const float* dW, const float* dX, const float* aux) {
  static const bool enabled = [] {
    const char* e = std::getenv("CNHIP_LINEAR_ONE_PASS");
    return !(e && e[0] == '0');
  }();
  const bool o_ok = O == 1 || O == 2 || O == 4 || O == 8 || O == 10 || O == 16;
  return enabled && o_ok && B % 512 == 0 && F % SK_FBLK == 0 && F / SK_FBLK <= 65535 &&
         B * F >= ((int64_t)1 << 22) && dW && X && dY && W && aligned16(X) && aligned16(dY) &&
         (!dX || aligned16(dX)) && (!aux || aligned16(aux));
}

// Rows per block (and per partial) of the one-pass backward
static int64_t skinny_rows(int64_t O) { return 256 * sk_rpl((int)O); }

// partials of the one-pass backward: per row chunk [F, O] then [O]
static size_t skinny_bytes(int64_t B, int64_t F, int64_t O) {
  return (size_t)((B / skinny_rows(O)) * (F * O + O)) * sizeof(float);
}

int linear_backward_skinny(const float* X, const float* W, const float* dY, float* dW, float* db,
                           float* dX, const float* aux, int64_t B, int64_t F, int64_t O,
                           int accumulate, int act, hipStream_t st, const char* who, bool* done) {
  *done = false;
  if (!skinny_serves(B, F, O, X, W, dY, dW, dX, act != 0 ? aux : nullptr)) return CNHIP_OK;
  CNHIP_REQUIRE(act >= 0 && act <= 2, "%s: bad activation %d", who, act);
  CNHIP_REQUIRE(act == 0 || (dX && aux), "%s: the activation derivative needs dX and its input", who);
  const int64_t chunks = B / skinny_rows(O), FO = F * O;
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
    switch (O) {
      case 1: skinny_launch_o<1>(st, act, sep, X, W, dY, aux, partial, dX, B, F); break;
      case 2: skinny_launch_o<2>(st, act, sep, X, W, dY, aux, partial, dX, B, F); break;
      case 4: skinny_launch_o<4>(st, act, sep, X, W, dY, aux, partial, dX, B, F); break;
      case 8: skinny_launch_o<8>(st, act, sep, X, W, dY, aux, partial, dX, B, F); break;
      case 10: skinny_launch_o<10>(st, act, sep, X, W, dY, aux, partial, dX, B, F); break;
      default: skinny_launch_o<16>(st, act, sep, X, W, dY, aux, partial, dX, B, F); break;
    }
    CNHIP_TRY(check_launch(who));
  }
  HbmTimer timer("skinny_reduce_kernel", 4.0 * (double)(chunks * (FO + O)) + (accumulate ? 8.0 : 4.0) * (double)(FO + O),
                 st);
  hipLaunchKernelGGL(skinny_reduce_kernel, dim3((unsigned)((FO + O + 255) / 256)), dim3(256), 0, st, partial, dW, db,
                     FO, (int)O, (int)chunks, accumulate);
  return check_launch(who);
}

// The one-pass forward above, when the shape is one it serves (O one of 1,
// 2, 4, 8, 10, 16; B % 256 == 0, F % 64 == 0, B F >= 2^20, X 16-byte
// aligned); *done says whether it ran.  Features per wave: the largest of
// 64, 32, 16 that still gives 512 blocks (else 16), so the partials stay few.
int linear_forward_skinny(const float* X, const float* W, const float* bias, float* Y, int64_t B, int64_t F,
                          int64_t O, hipStream_t st, const char* who, bool* done) {
  *done = false;
  const bool o_ok = O == 1 || O == 2 || O == 4 || O == 8 || O == 10 || O == 16;
  if (!(o_ok && B % 256 == 0 && F % 64 == 0 && B * F >= ((int64_t)1 << 20) && aligned16(X) && X && W && Y &&
        B / 256 <= 0x7fffffff && F / 64 <= 65535))
    return CNHIP_OK;
  int fw = 16;
  for (int c : {64, 32})
    if ((B / 256) * (F / (4 * c)) >= 512) {
      fw = c;
      break;
    }
  const int64_t chunks = F / (4 * fw), BO = B * O;
  void* ws = nullptr;
  CNHIP_TRY(scratch(st, kScratchGemm, (size_t)(chunks * BO) * sizeof(float), &ws, who));
  float* partial = static_cast<float*>(ws);
  *done = true;
  {
    HbmTimer timer("linear_fwd_skinny_kernel", 4.0 * ((double)B * F + (double)F * O + (double)(chunks * BO)), st);
    const dim3 grid((unsigned)(B / 256), (unsigned)chunks);
    switch (O) {
      case 1: hipLaunchKernelGGL(linear_fwd_skinny_kernel<1>, grid, dim3(256), 0, st, X, W, partial, B, F, fw); break;
      case 2: hipLaunchKernelGGL(linear_fwd_skinny_kernel<2>, grid, dim3(256), 0, st, X, W, partial, B, F, fw); break;
      case 4: hipLaunchKernelGGL(linear_fwd_skinny_kernel<4>, grid, dim3(256), 0, st, X, W, partial, B, F, fw); break;
      case 8: hipLaunchKernelGGL(linear_fwd_skinny_kernel<8>, grid, dim3(256), 0, st, X, W, partial, B, F, fw); break;
      case 10: hipLaunchKernelGGL(linear_fwd_skinny_kernel<10>, grid, dim3(256), 0, st, X, W, partial, B, F, fw); break;
      default: hipLaunchKernelGGL(linear_fwd_skinny_kernel<16>, grid, dim3(256), 0, st, X, W, partial, B, F, fw); break;
    }
    CNHIP_TRY(check_launch(who));
  }
  HbmTimer timer("linear_fwd_reduce_kernel", 4.0 * (double)(chunks * BO) + 4.0 * (double)BO, st);
  hipLaunchKernelGGL(linear_fwd_reduce_kernel, dim3((unsigned)((BO + 255) / 256)), dim3(256), 0, st, partial, bias, Y,
                     B, BO, (int)chunks);
  return check_launch(who);
}

// Largest GEMM-slot scratch request that cnhip_linear_backward_act makes for
// these arguments (its launches run in order on one stream, so one buffer of
// this size serves them all): the one-pass partials when that path serves
// the shape, else the split-K partials of the dW GEMM; and those of the dX
// GEMM unless the one-pass kernel wrote dX (it does for every act but the
// residual sum).
size_t linear_backward_act_scratch_bytes(const float* X, const float* W, const float* dY,
                                         const float* grad_W, const float* dX, const float* act_aux, int64_t B,
                                         int64_t I, int64_t O, int trainable, int act) {
  // the one pass with dX (act none, ReLU, GELU), else (act ReLU, GELU,
  // residual) the one pass for dW and db only, followed by the dX GEMM
  const bool run = trainable && B > 0;
  const bool full = run && act != CNHIP_ACT_RESIDUAL &&
                    skinny_serves(B, I, O, X, W, dY, grad_W, dX,
                                  act == CNHIP_ACT_RELU || act == CNHIP_ACT_GELU ? act_aux : nullptr);
  const bool one_pass =
      full || (run && act != CNHIP_ACT_NONE && skinny_serves(B, I, O, X, W, dY, grad_W, nullptr, nullptr));
  size_t need = one_pass ? skinny_bytes(B, I, O) : trainable ? gemm_scratch_bytes(1, 0, I, O, B, 1) : 0;
  if (dX && !full) need = std::max(need, gemm_scratch_bytes(0, 1, B, I, O, 1));
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
  bool one_pass = false;
  CNHIP_TRY(cnhip::linear_forward_skinny(X, W, b, Y, batch, in_features, out_features, cnhip::as_stream(stream),
                                         "cnhip_linear_forward", &one_pass));
  if (one_pass) return CNHIP_OK;
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
    // dW, db and dX in one launch when both products are small
    bool paired = false;
    CNHIP_TRY(cnhip::linear_backward_small_pair(X, W, dY, grad_W, grad_b, dX, batch, in_features, out_features,
                                                accumulate, st, who, &paired));
    if (paired) return CNHIP_OK;
    // dW[I,O] (+)= X^T[I,B] * dY[B,O]; db (+)= the column sums of dY (one
    // launch for both when the GEMM is small enough for the SIMT kernels)
    bool fused = false;
    CNHIP_TRY(cnhip::linear_wgrad_small(X, dY, grad_W, grad_b, batch, in_features, out_features, accumulate,
                                        st, who, &fused));
    if (!fused) {
      const cnhip::GemmSpec wgrad{1, 0, in_features, out_features, batch, 1.f, X, batch, 0, dY, batch, 0,
                                  beta, grad_W, in_features, 0, 1, nullptr, CNHIP_EPI_NONE, nullptr,
                                  nullptr, 0};
      if (dX) {
        // dX and dW in one launch where their tiles leave half the chip's block slots empty
        const cnhip::GemmSpec dgrad{0, 1, batch, in_features, out_features, 1.f, dY, batch, 0, W,
                                    in_features, 0, 0.f, dX, batch, 0, 1, nullptr, CNHIP_EPI_NONE,
                                    nullptr, nullptr, 0};
        CNHIP_TRY(cnhip::gemm_f32_pair(dgrad, wgrad, st, who, dY, grad_b, batch, out_features, accumulate));
        return CNHIP_OK;
      } else {
        CNHIP_TRY(cnhip::gemm_f32(1, 0, in_features, out_features, batch, 1.f, X, batch, dY, batch, beta,
                                  grad_W, in_features, nullptr, CNHIP_EPI_NONE, st, who));
      }
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
  if (act == CNHIP_ACT_NONE || batch == 0)
    return cnhip_linear_backward(X, W, dY, grad_W, grad_b, act == CNHIP_ACT_NONE ? dX : nullptr, batch,
                                 in_features, out_features, trainable, accumulate, stream);
  hipStream_t st = cnhip::as_stream(stream);
  // dX[B,I] = (dY W^T) * act'(act_aux), the activation's backward in the
  // epilogue; for the residual, dX = dY W^T + act_aux (the skip branch's gradient)
  const int epi = act == CNHIP_ACT_RELU   ? cnhip::EPI_DRELU
                  : act == CNHIP_ACT_GELU ? cnhip::EPI_DGELU
                                          : cnhip::EPI_ADD;
  CNHIP_REQUIRE(batch > 0 && in_features > 0 && out_features > 0, "%s: bad shape", who);
  const cnhip::GemmSpec dgrad{0, 1, batch, in_features, out_features, 1.f, dY, batch, 0, W, in_features, 0,
                              0.f, dX, batch, 0, 1, nullptr, epi, act_aux, nullptr, batch};
  if (trainable) {
    CNHIP_REQUIRE(grad_W != nullptr, "%s: trainable layer needs grad_W", who);
    bool fused = false;
    CNHIP_TRY(cnhip::linear_wgrad_small(X, dY, grad_W, grad_b, batch, in_features, out_features, accumulate,
                                        st, who, &fused));
    if (!fused) {
      // dX and dW in one launch where their tiles leave half the chip's block slots empty
      const cnhip::GemmSpec wgrad{1, 0, in_features, out_features, batch, 1.f, X, batch, 0, dY, batch, 0,
                                  accumulate ? 1.f : 0.f, grad_W, in_features, 0, 1, nullptr,
                                  CNHIP_EPI_NONE, nullptr, nullptr, 0};
      return cnhip::gemm_f32_pair(dgrad, wgrad, st, who, dY, grad_b, batch, out_features, accumulate);
    }
  }
  return cnhip::gemm_f32_act(0, 1, batch, in_features, out_features, dY, batch, W, in_features, dX,
                             batch, nullptr, epi, act_aux, nullptr, batch, st, who);
}

}  // extern "C"
