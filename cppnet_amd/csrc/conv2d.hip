// Conv2D as implicit GEMMs on the fp32 MFMA tile engine (mfma_core.hpp).
//
// ref: Conv2D::forward/backward, src/CppNet/layers/conv2d.cpp:78-198 (the
// semantics), conv2d_forward.cu:16-64 / conv2d_backward.cu:19-68 (the
// reference gpu path: one thread per output, atomicAdd scatter for grads).
//
// Tensors are ColMajor: X(n,c,h,w) = X[n + N*(c + C*(h + H*w))], so the batch
// index is the contiguous one, and W(oc,ic,kh,kw) = W[oc + OC*(ic + C*(kh +
// KS*kw))], i.e. W is a ColMajor [OC, K] matrix with k = ic + C*t, t = kh +
// KS*kw.  Hence, per output pixel (oh,ow):
//   forward  Y_pix[N, OC]  = A[N, K] * W^T       A(n,k) = X(n, ic, ih, iw) (0 if padded)
//   dgrad    dX_pix[N, C]  = A'[N, K'] * Wd      A'(n,k') = dY(n, oc, oh, ow), k' = oc + OC*t
//   wgrad    dW[OC, K | 1] = dY^T * [X | 1]      contraction over (n, pixel) pairs; the
//                                                extra ones-column yields the bias grad
// A and A' are gathered straight from HBM with float4 loads along the batch
// (contiguous), so no im2col buffer exists.  wgrad splits its long
// contraction over blocks and sums the partials in a fixed order.  Grads are
// overwritten, as the reference zeroes them first (conv2d.cpp:149-152).
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.hpp"
#include "mfma_core.hpp"

namespace cnhip {
namespace {

using mfma::BK;
using mfma::f32x16;
using mfma::f32x4;
using mfma::TileCfg;

using Cfg11 = TileCfg<1, 1, 1, 1>;  // 32 x 32, one wave
using CfgSN = TileCfg<4, 1, 1, 1>;  // 128 x 32
using CfgSM = TileCfg<1, 4, 1, 1>;  // 32 x 128
using CfgM = TileCfg<2, 2, 2, 1>;   // 128 x 64
using CfgS = TileCfg<2, 2, 1, 1>;   // 64 x 64
using CfgL = TileCfg<2, 2, 2, 2>;   // 128 x 128

struct ConvDims {
  int64_t N, C, H, W, OC, KS, S, P, HO, WO;
};

struct ConvArgs {
  ConvDims d;
  const float* X;     // forward / wgrad input
  const float* Wt;    // forward weights [OC, K]
  const float* Wd;    // dgrad weights relaid [K' = OC*T, C]
  const float* dY;    // dgrad / wgrad upstream grad
  const float* bias;  // forward bias or null
  float* out;         // Y (forward) / dX (dgrad)
  float* partial;     // wgrad split partials [splits][M*Ng]
  int64_t k_per_split;
  int has_bias;       // wgrad: adds the ones-column
  int nvec;           // N % 4 == 0 and the tensors read along n are 16-byte aligned
};

// Generic block loop: stage A/B tiles through LDS with the given loaders and
// accumulate.  LoadA/LoadB fill one float4 slot (rr, kk) of the tile.
template <class Cfg, bool AK, bool BKC, class LoadA, class LoadB>
__device__ __forceinline__ void igemm_mainloop(int64_t k_begin, int64_t k_end, LoadA&& la,
                                               LoadB&& lb, float* lds_a, float* lds_b,
                                               f32x16 (&acc)[Cfg::WM][Cfg::WN]) {
  using SA = mfma::TileSlots<AK, Cfg::BM, Cfg::NT>;
  using SB = mfma::TileSlots<BKC, Cfg::BN, Cfg::NT>;
  constexpr int TA = BK * Cfg::LDA, TB = BK * Cfg::LDB;
  f32x4 ra[SA::PER_THREAD], rb[SB::PER_THREAD];
  auto load = [&](int64_t k0) {
#pragma unroll
    for (int p = 0; p < SA::PER_THREAD; ++p) {
      int rr, kk;
      if (!SA::slot(p, rr, kk)) break;
      ra[p] = la(rr, k0 + kk);
    }
#pragma unroll
    for (int p = 0; p < SB::PER_THREAD; ++p) {
      int rr, kk;
      if (!SB::slot(p, rr, kk)) break;
      rb[p] = lb(rr, k0 + kk);
    }
  };
  const int ntiles = k_end > k_begin ? (int)((k_end - k_begin + BK - 1) / BK) : 0;
  if (ntiles > 0) {
    load(k_begin);
    SA::store(lds_a, ra);
    SB::store(lds_b, rb);
  }
  __syncthreads();
  for (int kt = 0; kt < ntiles; ++kt) {
    const int cur = kt & 1;
    const bool has_next = kt + 1 < ntiles;
    if (has_next) load(k_begin + (int64_t)(kt + 1) * BK);
    mfma::mfma_ktile<Cfg>(lds_a + cur * TA, lds_b + cur * TB, acc);
    if (has_next) {
      SA::store(lds_a + (cur ^ 1) * TA, ra);
      SB::store(lds_b + (cur ^ 1) * TB, rb);
    }
    __syncthreads();
  }
}

// float4 of X[base + n .. n+3] along the batch, zero past N.
__device__ __forceinline__ f32x4 load_n4(const float* __restrict__ base, int64_t n, int64_t N,
                                         bool vec) {
  if (vec && n + 3 < N) return *reinterpret_cast<const f32x4*>(base + n);
  f32x4 v;
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = (n + j < N) ? base[n + j] : 0.f;
  return v;
}

// ---------------------------------------------------------------- forward
template <class Cfg>
__global__ void __launch_bounds__(Cfg::NT) conv_fwd_kernel(ConvArgs a) {
  __shared__ float lds_a[2 * BK * Cfg::LDA];
  __shared__ float lds_b[2 * BK * Cfg::LDB];
  const ConvDims d = a.d;
  const int64_t K = d.C * d.KS * d.KS;
  const int nbm = (int)((d.N + Cfg::BM - 1) / Cfg::BM);
  const int64_t m0 = (int64_t)(blockIdx.x % nbm) * Cfg::BM;
  const int64_t n0 = (int64_t)(blockIdx.x / nbm) * Cfg::BN;
  const int64_t q = blockIdx.y, oh = q % d.HO, ow = q / d.HO;
  const bool vec = a.nvec;

  auto la = [&](int rr, int64_t k) -> f32x4 {
    if (k >= K) return f32x4{0.f, 0.f, 0.f, 0.f};
    const int64_t ic = k % d.C, t = k / d.C;
    const int64_t ih = oh * d.S - d.P + t % d.KS, iw = ow * d.S - d.P + t / d.KS;
    if (ih < 0 || ih >= d.H || iw < 0 || iw >= d.W) return f32x4{0.f, 0.f, 0.f, 0.f};
    return load_n4(a.X + d.N * (ic + d.C * (ih + d.H * iw)), m0 + rr, d.N, vec);
  };
  // B(k, oc) = W[oc + OC*k]: contiguous along oc
  auto lb = [&](int rr, int64_t k) -> f32x4 {
    const int64_t oc = n0 + rr;
    if (k >= K) return f32x4{0.f, 0.f, 0.f, 0.f};
    const float* base = a.Wt + d.OC * k;
    if ((d.OC & 3) == 0 && oc + 3 < d.OC) return *reinterpret_cast<const f32x4*>(base + oc);
    f32x4 v;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = (oc + j < d.OC) ? base[oc + j] : 0.f;
    return v;
  };
  f32x16 acc[Cfg::WM][Cfg::WN];
  mfma::zero_acc<Cfg>(acc);
  igemm_mainloop<Cfg, false, false>(0, K, la, lb, lds_a, lds_b, acc);

  float* Y = a.out + d.N * d.OC * q;  // Y_pix(n, oc) = Y[n + N*oc] at this pixel
  mfma::for_each_acc_run<Cfg>(acc, [&](int ml, int nl, const f32x4& v) {
    const int64_t n = m0 + ml, oc = n0 + nl;
    if (oc >= d.OC) return;
    const float b = a.bias ? a.bias[oc] : 0.f;
    if (vec && n + 3 < d.N) {
      f32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = a.bias ? v[e] + b : v[e];
      *reinterpret_cast<f32x4*>(Y + n + d.N * oc) = o;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (n + e < d.N) Y[n + e + d.N * oc] = a.bias ? v[e] + b : v[e];
    }
  });
}

// ---------------------------------------------------------------- dgrad
// Wd[k' + K'*ic] = W[oc + OC*(ic + C*t)], k' = oc + OC*t
__global__ void __launch_bounds__(256) conv_relayout_w_kernel(const float* __restrict__ Wt,
                                                              float* __restrict__ Wd, int64_t OC,
                                                              int64_t C, int64_t T) {
  const int64_t total = OC * C * T, Kp = OC * T;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t oc = i % OC, ic = (i / OC) % C, t = i / (OC * C);
    Wd[(oc + OC * t) + Kp * ic] = Wt[i];
  }
}

template <class Cfg>
__global__ void __launch_bounds__(Cfg::NT) conv_dgrad_kernel(ConvArgs a) {
  __shared__ float lds_a[2 * BK * Cfg::LDA];
  __shared__ float lds_b[2 * BK * Cfg::LDB];
  const ConvDims d = a.d;
  const int64_t T = d.KS * d.KS, Kp = d.OC * T;
  const int nbm = (int)((d.N + Cfg::BM - 1) / Cfg::BM);
  const int64_t m0 = (int64_t)(blockIdx.x % nbm) * Cfg::BM;
  const int64_t n0 = (int64_t)(blockIdx.x / nbm) * Cfg::BN;
  const int64_t q = blockIdx.y, h = q % d.H, w = q / d.H;
  const bool vec = a.nvec;

  // A'(n, k') = dY(n, oc, oh, ow) where (oh, ow) is the output pixel whose
  // tap t = kh + KS*kw reads input (h, w): oh*S - P + kh = h.
  auto la = [&](int rr, int64_t k) -> f32x4 {
    if (k >= Kp) return f32x4{0.f, 0.f, 0.f, 0.f};
    const int64_t oc = k % d.OC, t = k / d.OC;
    const int64_t ohn = h + d.P - t % d.KS, own = w + d.P - t / d.KS;
    if (ohn < 0 || own < 0 || ohn % d.S != 0 || own % d.S != 0) return f32x4{0.f, 0.f, 0.f, 0.f};
    const int64_t oh = ohn / d.S, ow = own / d.S;
    if (oh >= d.HO || ow >= d.WO) return f32x4{0.f, 0.f, 0.f, 0.f};
    return load_n4(a.dY + d.N * (oc + d.OC * (oh + d.HO * ow)), m0 + rr, d.N, vec);
  };
  // B(k', ic) = Wd[k' + K'*ic]: contiguous along k'
  auto lb = [&](int rr, int64_t k) -> f32x4 {
    const int64_t ic = n0 + rr;
    if (ic >= d.C) return f32x4{0.f, 0.f, 0.f, 0.f};
    const float* base = a.Wd + Kp * ic;
    if ((Kp & 3) == 0 && k + 3 < Kp) return *reinterpret_cast<const f32x4*>(base + k);
    f32x4 v;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = (k + j < Kp) ? base[k + j] : 0.f;
    return v;
  };
  f32x16 acc[Cfg::WM][Cfg::WN];
  mfma::zero_acc<Cfg>(acc);
  igemm_mainloop<Cfg, false, true>(0, Kp, la, lb, lds_a, lds_b, acc);

  float* dX = a.out + d.N * d.C * q;
  mfma::for_each_acc_run<Cfg>(acc, [&](int ml, int nl, const f32x4& v) {
    const int64_t n = m0 + ml, ic = n0 + nl;
    if (ic >= d.C) return;
    if (vec && n + 3 < d.N) {
      *reinterpret_cast<f32x4*>(dX + n + d.N * ic) = v;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (n + e < d.N) dX[n + e + d.N * ic] = v[e];
    }
  });
}

// ---------------------------------------------------------------- wgrad
// M = OC, Ng = C*T (+1 ones-column for the bias), contraction index
// k = n + N*q over (sample, output pixel); split over blockIdx.z.
template <class Cfg>
__global__ void __launch_bounds__(Cfg::NT) conv_wgrad_kernel(ConvArgs a) {
  __shared__ float lds_a[2 * BK * Cfg::LDA];
  __shared__ float lds_b[2 * BK * Cfg::LDB];
  const ConvDims d = a.d;
  const int64_t CT = d.C * d.KS * d.KS, Ng = CT + a.has_bias, Kc = d.N * d.HO * d.WO;
  const int nbm = (int)((d.OC + Cfg::BM - 1) / Cfg::BM);
  const int64_t m0 = (int64_t)(blockIdx.x % nbm) * Cfg::BM;
  const int64_t n0 = (int64_t)(blockIdx.x / nbm) * Cfg::BN;
  const int64_t k_begin = (int64_t)blockIdx.z * a.k_per_split;
  const int64_t k_end = min(Kc, k_begin + a.k_per_split);
  // float4s along k stay inside one output pixel when N % 4 == 0 (k starts at
  // multiples of 4)
  const bool vec = a.nvec;

  // A(oc, k) = dY[n + N*(oc + OC*q)]
  auto la = [&](int rr, int64_t k) -> f32x4 {
    const int64_t oc = m0 + rr;
    f32x4 v{0.f, 0.f, 0.f, 0.f};
    if (oc >= d.OC) return v;
    if (vec && k + 3 < k_end) {
      const int64_t n = k % d.N, q = k / d.N;
      return *reinterpret_cast<const f32x4*>(a.dY + n + d.N * (oc + d.OC * q));
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t kj = k + j;
      if (kj < k_end) v[j] = a.dY[kj % d.N + d.N * (oc + d.OC * (kj / d.N))];
    }
    return v;
  };
  // B(k, j) = X(n, ic, ih, iw) for j = ic + C*t < CT; 1 for the bias column
  auto lb = [&](int rr, int64_t k) -> f32x4 {
    const int64_t j = n0 + rr;
    f32x4 v{0.f, 0.f, 0.f, 0.f};
    if (j >= Ng) return v;
    if (j == CT) {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (k + e < k_end) ? 1.f : 0.f;
      return v;
    }
    const int64_t ic = j % d.C, t = j / d.C, kh = t % d.KS, kw = t / d.KS;
    if (vec && k + 3 < k_end) {
      const int64_t n = k % d.N, q = k / d.N;
      const int64_t ih = (q % d.HO) * d.S - d.P + kh, iw = (q / d.HO) * d.S - d.P + kw;
      if (ih < 0 || ih >= d.H || iw < 0 || iw >= d.W) return v;
      return *reinterpret_cast<const f32x4*>(a.X + n + d.N * (ic + d.C * (ih + d.H * iw)));
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t kj = k + e;
      if (kj >= k_end) break;
      const int64_t n = kj % d.N, q = kj / d.N;
      const int64_t ih = (q % d.HO) * d.S - d.P + kh, iw = (q / d.HO) * d.S - d.P + kw;
      if (ih >= 0 && ih < d.H && iw >= 0 && iw < d.W)
        v[e] = a.X[n + d.N * (ic + d.C * (ih + d.H * iw))];
    }
    return v;
  };
  f32x16 acc[Cfg::WM][Cfg::WN];
  mfma::zero_acc<Cfg>(acc);
  igemm_mainloop<Cfg, true, true>(k_begin, k_end, la, lb, lds_a, lds_b, acc);

  float* P = a.partial + (int64_t)blockIdx.z * d.OC * Ng;
  mfma::for_each_acc_run<Cfg>(acc, [&](int ml, int nl, const f32x4& v) {
    const int64_t m = m0 + ml, j = n0 + nl;
    if (j >= Ng) return;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (m + e < d.OC) P[(m + e) + d.OC * j] = v[e];
  });
}

// gW[oc + OC*j] = sum_z partial[z][oc + OC*j]; the ones-column goes to gb.
// 64 consecutive outputs per block (coalesced along e); the RW waves of a
// block each sum one contiguous chunk of z in ascending order, and the chunk
// sums are added in ascending order: a fixed summation order for any launch.
constexpr int WGRAD_RW = 16;
__global__ void __launch_bounds__(64 * WGRAD_RW) conv_wgrad_reduce_kernel(
    const float* __restrict__ partial, int splits, int64_t OC, int64_t CT, int has_bias,
    float* __restrict__ gW, float* __restrict__ gb) {
  __shared__ float part[WGRAD_RW][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t Ng = CT + has_bias, total = OC * Ng;
  const int64_t e = (int64_t)blockIdx.x * 64 + lane;
  const int per = (splits + WGRAD_RW - 1) / WGRAD_RW;
  const int z0 = w * per, z1 = min(splits, z0 + per);
  float s = 0.f;
  if (e < total)
    for (int z = z0; z < z1; ++z) s += partial[(int64_t)z * total + e];
  part[w][lane] = s;
  __syncthreads();
  if (w == 0 && e < total) {
    float t = part[0][lane];
#pragma unroll
    for (int i = 1; i < WGRAD_RW; ++i) t += part[i][lane];
    const int64_t j = e / OC;
    if (j < CT) gW[e] = t;
    else if (gb) gb[e - OC * CT] = t;
  }
}

int check_dims(const ConvDims& d, const char* who) {
  CNHIP_REQUIRE(d.N > 0 && d.C > 0 && d.H > 0 && d.W > 0 && d.OC > 0 && d.KS > 0 && d.S > 0 &&
                    d.P >= 0,
                "%s: bad shape N=%lld C=%lld H=%lld W=%lld OC=%lld KS=%lld S=%lld P=%lld", who,
                (long long)d.N, (long long)d.C, (long long)d.H, (long long)d.W, (long long)d.OC,
                (long long)d.KS, (long long)d.S, (long long)d.P);
  CNHIP_REQUIRE(d.HO > 0 && d.WO > 0, "%s: kernel %lld larger than the padded input", who,
                (long long)d.KS);
  CNHIP_REQUIRE(d.HO * d.WO <= 65535 && d.H * d.W <= 65535,
                "%s: %lld x %lld pixels exceed the 65535-pixel grid limit", who, (long long)d.H,
                (long long)d.W);
  return CNHIP_OK;
}

ConvDims make_dims(int64_t N, int64_t C, int64_t H, int64_t W, int64_t OC, int64_t KS, int64_t S,
                   int64_t P) {
  ConvDims d{N, C, H, W, OC, KS, S, P, 0, 0};
  if (S > 0) {
    d.HO = (H + 2 * P - KS) / S + 1;
    d.WO = (W + 2 * P - KS) / S + 1;
  }
  return d;
}

// Tile shape for an (M rows along the batch) x (Ng channels) per-pixel GEMM.
template <template <class> class Kern>
void launch_pixel(const ConvArgs& a, int64_t M, int64_t Ng, int64_t pixels, hipStream_t st) {
  auto go = [&](auto cfg) {
    using Cfg = decltype(cfg);
    const int64_t tiles = ((M + Cfg::BM - 1) / Cfg::BM) * ((Ng + Cfg::BN - 1) / Cfg::BN);
    // algorithmic flops: 2 * N * (output pixels) * OC * C * KS^2 for both directions
    const ConvDims& d = a.d;
    TimingRec* rec = timing_slot(2.0 * d.N * d.HO * d.WO * d.OC * d.C * d.KS * d.KS);
    if (rec) (void)hipEventRecord(rec->start, st);
    hipLaunchKernelGGL(Kern<Cfg>::fn(), dim3((unsigned)tiles, (unsigned)pixels), dim3(Cfg::NT), 0,
                       st, a);
    if (rec) (void)hipEventRecord(rec->stop, st);
  };
  if (Ng <= 32) go(CfgSN{});
  else if (Ng <= 64) go(CfgM{});
  else go(CfgL{});
}

template <class Cfg>
struct FwdK {
  static auto fn() { return &conv_fwd_kernel<Cfg>; }
};
template <class Cfg>
struct DgradK {
  static auto fn() { return &conv_dgrad_kernel<Cfg>; }
};

}  // namespace
}  // namespace cnhip

using cnhip::as_stream;

extern "C" {

int cnhip_conv2d_forward(const float* X, const float* W, const float* b, float* Y, int64_t N,
                         int64_t C, int64_t H, int64_t Wd, int64_t OC, int64_t KS, int64_t S,
                         int64_t P, cnhip_stream_t stream) {
  const char* who = "cnhip_conv2d_forward";
  const cnhip::ConvDims d = cnhip::make_dims(N, C, H, Wd, OC, KS, S, P);
  CNHIP_TRY(cnhip::check_dims(d, who));
  CNHIP_REQUIRE(X && W && Y, "%s: NULL pointer", who);
  cnhip::ConvArgs a{};
  a.d = d; a.X = X; a.Wt = W; a.bias = b; a.out = Y;
  a.nvec = (N % 4 == 0) && cnhip::aligned16(X) && cnhip::aligned16(Y);
  cnhip::launch_pixel<cnhip::FwdK>(a, N, OC, d.HO * d.WO, as_stream(stream));
  return cnhip::check_launch(who);
}

int cnhip_conv2d_backward(const float* X, const float* W, const float* dY, float* gW, float* gb,
                          float* dX, int64_t N, int64_t C, int64_t H, int64_t Wd, int64_t OC,
                          int64_t KS, int64_t S, int64_t P, cnhip_stream_t stream) {
  const char* who = "cnhip_conv2d_backward";
  const cnhip::ConvDims d = cnhip::make_dims(N, C, H, Wd, OC, KS, S, P);
  CNHIP_TRY(cnhip::check_dims(d, who));
  CNHIP_REQUIRE(X && W && dY && gW, "%s: NULL pointer", who);
  hipStream_t st = as_stream(stream);
  const int64_t T = KS * KS, CT = C * T;

  // ---- weight + bias grads: split-K implicit GEMM, then a fixed-order sum
  cnhip::ConvArgs a{};
  a.d = d; a.X = X; a.dY = dY;
  a.has_bias = gb ? 1 : 0;
  a.nvec = (N % 4 == 0) && cnhip::aligned16(X) && cnhip::aligned16(dY);
  const int64_t Ng = CT + a.has_bias, Kc = N * d.HO * d.WO;
  auto wgrad = [&](auto cfg) -> int {
    using Cfg = decltype(cfg);
    const int64_t tiles = ((OC + Cfg::BM - 1) / Cfg::BM) * ((Ng + Cfg::BN - 1) / Cfg::BN);
    int64_t splits = std::max<int64_t>(1, (1024 + tiles - 1) / tiles);
    splits = std::min<int64_t>(splits, std::max<int64_t>(1, Kc / (8 * cnhip::mfma::BK)));
    int64_t kps = (Kc + splits - 1) / splits;
    kps = (kps + cnhip::mfma::BK - 1) / cnhip::mfma::BK * cnhip::mfma::BK;
    splits = (Kc + kps - 1) / kps;
    a.k_per_split = kps;
    void* ws = nullptr;
    CNHIP_TRY(cnhip::check_hip(hipMallocAsync(&ws, (size_t)splits * OC * Ng * sizeof(float), st), who));
    a.partial = static_cast<float*>(ws);
    cnhip::TimingRec* rec = cnhip::timing_slot(2.0 * N * d.HO * d.WO * OC * CT);
    if (rec) (void)hipEventRecord(rec->start, st);
    hipLaunchKernelGGL(cnhip::conv_wgrad_kernel<Cfg>, dim3((unsigned)tiles, 1, (unsigned)splits),
                       dim3(Cfg::NT), 0, st, a);
    int status = cnhip::check_launch(who);
    if (rec) (void)hipEventRecord(rec->stop, st);
    if (status == CNHIP_OK) {
      hipLaunchKernelGGL(cnhip::conv_wgrad_reduce_kernel, dim3((unsigned)((OC * Ng + 63) / 64)),
                         dim3(64 * cnhip::WGRAD_RW), 0, st, a.partial, (int)splits, OC, CT,
                         a.has_bias, gW, gb);
      status = cnhip::check_launch(who);
    }
    const int st2 = cnhip::check_hip(hipFreeAsync(ws, st), who);
    return status != CNHIP_OK ? status : st2;
  };
  int status;
  if (OC <= 32) status = Ng <= 32 ? wgrad(cnhip::Cfg11{}) : wgrad(cnhip::CfgSM{});
  else if (OC <= 64) status = wgrad(cnhip::CfgS{});
  else status = wgrad(cnhip::CfgL{});
  CNHIP_TRY(status);

  // ---- input grad: relay W out as [OC*T, C], then per-input-pixel GEMMs
  if (dX) {
    void* ws = nullptr;
    CNHIP_TRY(cnhip::check_hip(hipMallocAsync(&ws, (size_t)OC * CT * sizeof(float), st), who));
    float* Wr = static_cast<float*>(ws);
    hipLaunchKernelGGL(cnhip::conv_relayout_w_kernel, dim3(cnhip::elementwise_grid(OC * CT, 256)),
                       dim3(256), 0, st, W, Wr, OC, C, T);
    status = cnhip::check_launch(who);
    if (status == CNHIP_OK) {
      cnhip::ConvArgs b{};
      b.d = d; b.dY = dY; b.Wd = Wr; b.out = dX;
      b.nvec = (N % 4 == 0) && cnhip::aligned16(dY) && cnhip::aligned16(dX);
      cnhip::launch_pixel<cnhip::DgradK>(b, N, C, H * Wd, st);
      status = cnhip::check_launch(who);
    }
    const int st2 = cnhip::check_hip(hipFreeAsync(ws, st), who);
    CNHIP_TRY(status);
    CNHIP_TRY(st2);
  }
  return CNHIP_OK;
}

}  // extern "C"
