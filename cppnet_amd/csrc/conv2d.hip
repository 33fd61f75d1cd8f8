// Conv2D as implicit GEMMs on the fp32 MFMA tile engine (mfma_kpack.hpp).
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
// Forward and dgrad run one GEMM per pixel (blocks in XCD-contiguous order, below).  With the pixel
// fixed, A's column k is one fixed element offset of X (dY), or padding; a
// table of those offsets is built in LDS once per block, so the K loop does
// no index arithmetic: a 16-byte unit of A (4 samples at one k) is one table
// read and one float4 along the batch.  No im2col buffer exists.  wgrad contracts over k = n + N*q; when N is a multiple of
// the k-tile depth, a k-tile lies inside one output pixel q, so both of its
// operands are plain k-contiguous float4 loads with one decode per tile.
// wgrad splits its long contraction over blocks (and, for small tiles, over
// the waves of a block) and sums the partials in a fixed order.  Grads are
// overwritten, as the reference zeroes them first (conv2d.cpp:149-152).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "act_math.hpp"
#include "common.hpp"
#include "mfma_kpack.hpp"

namespace cnhip {
namespace {

using kp::f32x16;
using kp::f32x4;

struct ConvDims {
  int64_t N, C, H, W, OC, KS, S, P, HO, WO;
};

struct ConvArgs {
  ConvDims d;
  const float* src;   // gathered operand: X (forward, wgrad) / dY (dgrad)
  const float* wt;    // forward W [OC, K] / dgrad Wd [K', C] (k-contiguous rows)
  const float* dY;    // wgrad A
  const float* bias;  // forward bias or null
  float* out;         // Y (forward) / dX (dgrad)
  float* partial;     // wgrad split partials [splits][OC * Ng]
  int64_t k_per_split;
  int relu;           // forward: ReLU in the epilogue
  int has_bias;       // wgrad: adds the ones-column
  int out_vec;        // N % 4 == 0 and out 16-byte aligned
  int src_vec;        // forward / dgrad: N % 4 == 0 and src 16-byte aligned
  int wt_vec;         // forward: OC % 4 == 0, dgrad: K' % 4 == 0; weights 16-byte aligned
  int aligned;        // wgrad: N % KT == 0 and X, dY 16-byte aligned
  // wgrad through a ReLU -> MaxPool2D (pool > 0): dY is the pooled gradient
  // [N, OC, HP, WP], pidx its int32 argmax and pout the pooled output
  const int32_t* pidx;
  const float* pout;
  int pool;
  int64_t HP;
};

// Capacity of the per-block gather table (ints, 18 KiB of LDS).
constexpr int KTBL = 4608;

// Element offset of A(0, k) in the gathered tensor at pixel (q1, q2), or -1
// where the term is zero.  Forward: X at output pixel (oh, ow) = (q1, q2);
// dgrad: dY at input pixel (h, w) = (q1, q2), where output pixel (oh, ow)
// reads (h, w) through tap t = kh + KS*kw when oh*S - P + kh = h.
template <bool DGRAD, class I>
__device__ __forceinline__ I gather_off(const ConvDims& d, I q1, I q2, I k) {
  if (!DGRAD) {
    const I C = (I)d.C, KS = (I)d.KS;
    const I ic = k % C, t = k / C;
    const I ih = q1 * (I)d.S - (I)d.P + t % KS, iw = q2 * (I)d.S - (I)d.P + t / KS;
    if (ih < 0 || ih >= (I)d.H || iw < 0 || iw >= (I)d.W) return -1;
    return (I)d.N * (ic + C * (ih + (I)d.H * iw));
  }
  const I OC = (I)d.OC, KS = (I)d.KS, S = (I)d.S;
  const I oc = k % OC, t = k / OC;
  const I ohn = q1 + (I)d.P - t % KS, own = q2 + (I)d.P - t / KS;
  if (ohn < 0 || own < 0 || ohn % S != 0 || own % S != 0) return -1;
  const I oh = ohn / S, ow = own / S;
  if (oh >= (I)d.HO || ow >= (I)d.WO) return -1;
  return (I)d.N * (oc + OC * (oh + (I)d.HO * ow));
}

// Hardware dispatch deals consecutive block ids to the 8 XCDs in turn, and
// each XCD has its own L2.  This maps a linear block id so that each XCD
// owns a contiguous range of logical blocks: consecutive output pixels (or
// the k-splits of neighbouring pixels), whose 3x3 neighbourhoods overlap,
// then share that XCD's L2 instead of each XCD fetching its own copy.
__device__ __forceinline__ int xcd_contiguous(int bid, int total) {
  const int xcd = bid & 7, local = bid >> 3;
  const int base = total >> 3, rem = total & 7;
  return xcd * base + min(xcd, rem) + local;
}

// ------------------------------------------------------- forward / dgrad
// Stage for kp::pipeline.  A(n, k) = src[n + off(k)] (rows contiguous along
// the batch: a unit is 4 consecutive samples at one k, one table lookup and
// one float4 when N % 4 == 0); B = W (forward: B(oc, k) = W[oc + OC*k],
// contiguous along oc) or Wd (dgrad: B(ic, k) = Wd[k + K'*ic], contiguous
// along k).
template <class C, bool DGRAD, bool TBL, bool FAST>
struct PixelStage {
  using OA = kp::Operand<false, C::BM, C::NT, C::KT>;
  using OB = kp::Operand<DGRAD, C::BN, C::NT, C::KT>;
  const ConvArgs& a;
  const int* tbl;
  int64_t m0, n0, K, q1, q2;
  f32x4 ra[2][OA::REGS], rb[2][OB::REGS];

  __device__ PixelStage(const ConvArgs& a_, const int* tbl_, int64_t m0_, int64_t n0_, int64_t K_,
                        int64_t q1_, int64_t q2_)
      : a(a_), tbl(tbl_), m0(m0_), n0(n0_), K(K_), q1(q1_), q2(q2_) {}

  template <int S>
  __device__ __forceinline__ void load(int t) {
    const ConvDims& d = a.d;
    const int64_t k0 = (int64_t)t * C::KT;
#pragma unroll
    for (int p = 0; p < OA::PER; ++p) {
      int r, k;
      if (!OA::origin(p, r, k)) break;
      const int64_t row = m0 + r, gk = k0 + k;
      // table padded with -1 up to a whole number of k-tiles
      const int64_t o = TBL ? (int64_t)tbl[gk] : (gk < K ? gather_off<DGRAD, int64_t>(d, q1, q2, gk) : -1);
      f32x4 v{0.f, 0.f, 0.f, 0.f};
      if (o >= 0) {
        if (a.src_vec && (FAST || row + 3 < d.N)) {
          v = *reinterpret_cast<const f32x4*>(a.src + o + row);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (row + j < d.N) v[j] = a.src[o + row + j];
        }
      }
      ra[S][p] = v;
    }
    if (DGRAD)
      OB::template load<FAST>(a.wt, K, n0, k0, d.C, K, rb[S]);
    else
      OB::template load<FAST>(a.wt, d.OC, n0, k0, d.OC, K, rb[S]);
  }
  template <int S>
  __device__ __forceinline__ void store(float* buf) {
    OA::store(buf, ra[S]);
    OB::store(buf + OA::FLOATS, rb[S]);
  }
};

template <class C, bool DGRAD, bool TBL>
__global__ void __launch_bounds__(C::NT) conv_pixel_kernel(ConvArgs a) {
  constexpr int FLOATS = 2 * kp::stage_floats<PixelStage<C, DGRAD, TBL, true>>();
  __shared__ __align__(16) float lds[FLOATS];
  __shared__ __align__(16) int tbl[TBL ? KTBL : 4];
  static_assert((C::WGK - 1) * C::WGM * C::WGN * C::WM * C::WN * 1024 <= FLOATS,
                "reduce_wgk needs more LDS than the operand buffers");
  const ConvDims& d = a.d;
  const int64_t Ng = DGRAD ? d.C : d.OC;
  const int64_t K = (DGRAD ? d.OC : d.C) * d.KS * d.KS;
  const int nbm = (int)((d.N + C::BM - 1) / C::BM);
  // gridDim.x tiles per pixel, gridDim.y pixels
  const int lb = xcd_contiguous((int)(blockIdx.x + gridDim.x * blockIdx.y), (int)(gridDim.x * gridDim.y));
  const int tile = lb % (int)gridDim.x;
  const int64_t m0 = (int64_t)(tile % nbm) * C::BM;
  const int64_t n0 = (int64_t)(tile / nbm) * C::BN;
  const int64_t q = lb / (int)gridDim.x, HQ = DGRAD ? d.H : d.HO;
  const int64_t q1 = q % HQ, q2 = q / HQ;
  const int ntiles = (int)((K + C::KT - 1) / C::KT);
  if (TBL) {  // host guarantees ntiles * KT <= KTBL and 32-bit offsets
    for (int k = threadIdx.x; k < ntiles * C::KT; k += C::NT)
      tbl[k] = k < K ? gather_off<DGRAD, int>(d, (int)q1, (int)q2, k) : -1;
    __syncthreads();
  }
  const bool fast = m0 + C::BM <= d.N && n0 + C::BN <= Ng && K % C::KT == 0 && a.wt_vec;
  f32x16 acc[C::WM][C::WN];
  kp::zero_acc<C>(acc);
  if (fast) {
    PixelStage<C, DGRAD, TBL, true> s(a, tbl, m0, n0, K, q1, q2);
    kp::pipeline<C>(ntiles, lds, s, acc);
  } else {
    PixelStage<C, DGRAD, TBL, false> s(a, tbl, m0, n0, K, q1, q2);
    kp::pipeline<C>(ntiles, lds, s, acc);
  }
  kp::reduce_wgk<C>(lds, acc);

  float* out = a.out + d.N * Ng * q;  // out_pix(n, c) = out[n + N*c]
  kp::for_each_acc_run<C>(acc, [&](int ml, int nl, const f32x4& v) {
    const int64_t n = m0 + ml, c = n0 + nl;
    if (c >= Ng) return;
    f32x4 o = v;
    if (!DGRAD) {
      if (a.bias) {
        const float b = a.bias[c];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = v[e] + b;
      }
      if (a.relu) {
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = relu_f(o[e]);
      }
    }
    if (a.out_vec && n + 3 < d.N) {
      *reinterpret_cast<f32x4*>(out + n + d.N * c) = o;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (n + e < d.N) out[n + e + d.N * c] = o[e];
    }
  });
}

// ------------------------------------------------------- short-contraction forward
// Forward of a convolution whose contraction is short (C KS^2 <= 32, such as
// an RGB input layer's 27): 2 C KS^2 flops per output against the 4 bytes of
// writing it, so the layer is bound by writing Y, and the per-pixel MFMA
// tile above spends its time staging two k-tiles through LDS.  Here the
// operands go straight from memory into MFMA registers: a block takes one
// output pixel and 256 samples, each of its 4 waves 64 samples x all output
// channels in chunks of 32, over k-steps of 4 taps (v_mfma_f32_16x16x4f32;
// taps past C KS^2 and padded taps are 0).  The weights are the row operand
// (16 channels per row tile) and X the column operand: column tile nt holds
// samples n0 + 4 r + nt (r = 0..15), so a lane loads its four column tiles'
// operands at one tap as one float4 of X, and an output row (one channel)
// comes back as float4s of 4 consecutive samples, lanes r = 0..15 covering
// 256 contiguous bytes: every store instruction writes whole cache lines.
// Taps are summed in ascending k = ic + C (kh + KS kw), then the bias is
// added, then the ReLU, as in the MFMA epilogue.  The grid is 2 blocks per
// CU (512 blocks of 256 samples), each looping over every gridDim.x-th
// pixel: one block per pixel (1024 at config 3, 3 resident per CU) had left
// the last third of the CUs' slots a whole extra round.
constexpr int kDirectMaxK = 32;

__global__ void __launch_bounds__(256) conv_direct_fwd_kernel(ConvArgs a) {
  const ConvDims& d = a.d;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane >> 4, r = lane & 15;
  const int K = (int)(d.C * d.KS * d.KS), OC = (int)d.OC, npix = (int)(d.HO * d.WO);
  __shared__ int off[kDirectMaxK];  // element offset of X(0, tap k), or -1 (padding, k >= K)
  const int64_t n0 = (int64_t)blockIdx.y * 256 + 64 * wave;  // N % 64 == 0
  // the grid holds as many blocks as the CUs run at once; each takes every
  // gridDim.x-th pixel, so every CU gets the same number of pixels
  for (int pix = (int)blockIdx.x; pix < npix; pix += (int)gridDim.x) {
    // 32-bit index arithmetic (the host checks that X's offsets fit): 64-bit
    // division has no instruction and expands into long sequences
    const int oh = pix % (int)d.HO, ow = pix / (int)d.HO;
    __syncthreads();  // the previous pixel's offsets have been read
    if (threadIdx.x < kDirectMaxK)
      off[threadIdx.x] = (int)threadIdx.x < K ? gather_off<false, int>(d, oh, ow, (int)threadIdx.x) : -1;
    __syncthreads();
    if (n0 >= d.N) continue;
    f32x4 xv[kDirectMaxK / 4];  // X(n0 + 4 r .. 4 r + 3, tap 4 ks + q)
#pragma unroll
    for (int ks = 0; ks < kDirectMaxK / 4; ++ks) {
      const int o = off[4 * ks + q];
      xv[ks] = o >= 0 ? *reinterpret_cast<const f32x4*>(a.src + o + n0 + 4 * r) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const int nks = (K + 3) / 4;
    for (int oc0 = 0; oc0 < OC; oc0 += 32) {
      float wv[2][kDirectMaxK / 4];  // W(oc0 + 16 mt + r, tap 4 ks + q)
#pragma unroll
      for (int ks = 0; ks < kDirectMaxK / 4; ++ks)
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const int k = 4 * ks + q;
          wv[mt][ks] = k < K ? a.wt[oc0 + 16 * mt + r + (int64_t)OC * k] : 0.f;
        }
      f32x4 acc[2][4];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < kDirectMaxK / 4; ++ks)
        if (ks < nks) {
#pragma unroll
          for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int nt = 0; nt < 4; ++nt)
              acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[mt][ks], xv[ks][nt], acc[mt][nt], 0, 0, 0);
        }
      // acc[mt][nt][i]: channel oc0 + 16 mt + 4 q + i, sample n0 + 4 r + nt
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int64_t oc = oc0 + 16 * mt + 4 * q + i;
          f32x4 o;
#pragma unroll
          for (int nt = 0; nt < 4; ++nt) o[nt] = acc[mt][nt][i];
          if (a.bias) {
            const float b = a.bias[oc];
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = o[e] + b;
          }
          if (a.relu) {
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = relu_f(o[e]);
          }
          *reinterpret_cast<f32x4*>(a.out + n0 + 4 * r + d.N * (oc + d.OC * pix)) = o;
        }
    }
  }
}

// conv_direct_fwd_kernel with the ReLU and a MaxPool2D (window p x p,
// stride p, windows tiling the conv output) fused in: a block takes one
// pooled pixel and 256 samples, and each wave runs the direct kernel's MFMAs
// (same operands, same order) for the p^2 conv pixels of the window in the
// pool's (ph, pw) order, keeping per output the running maximum and its
// window index ph p + pw -- strict >, from -inf and index 0, as
// maxpool_fwd_vec_kernel compares -- so the pooled output and the argmax are
// bit for bit those of the two launches, and the conv output is never
// written.  The next conv pixel's X operands are loaded before the current
// one's MFMAs.
constexpr int kPoolMaxFused = 4;
typedef int i32x4 __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(256) conv_direct_pool_fwd_kernel(ConvArgs a, int pool, float* __restrict__ P,
                                                                   int32_t* __restrict__ pidx) {
  const ConvDims& d = a.d;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane >> 4, r = lane & 15;
  const int K = (int)(d.C * d.KS * d.KS), OC = (int)d.OC;
  const int HP = (int)d.HO / pool, npp = HP * ((int)d.WO / pool), nsub = pool * pool;
  __shared__ int off[kPoolMaxFused * kPoolMaxFused][kDirectMaxK];  // per window tap s = ph pool + pw
  const int64_t n0 = (int64_t)blockIdx.y * 256 + 64 * wave;  // N % 64 == 0
  const int nks = (K + 3) / 4;
  for (int pp = (int)blockIdx.x; pp < npp; pp += (int)gridDim.x) {
    const int py = pp % HP, px = pp / HP;
    __syncthreads();  // the previous window's offsets have been read
    for (int e = (int)threadIdx.x; e < nsub * kDirectMaxK; e += 256) {
      const int sub = e / kDirectMaxK, k = e % kDirectMaxK;
      off[sub][k] = k < K ? gather_off<false, int>(d, py * pool + sub / pool, px * pool + sub % pool, k) : -1;
    }
    __syncthreads();
    if (n0 >= d.N) continue;
    auto load_x = [&](int sub, f32x4 (&xv)[kDirectMaxK / 4]) {  // X(n0 + 4 r .. 4 r + 3, tap 4 ks + q)
#pragma unroll
      for (int ks = 0; ks < kDirectMaxK / 4; ++ks) {
        const int o = off[sub][4 * ks + q];
        xv[ks] = o >= 0 ? *reinterpret_cast<const f32x4*>(a.src + o + n0 + 4 * r) : f32x4{0.f, 0.f, 0.f, 0.f};
      }
    };
    for (int oc0 = 0; oc0 < OC; oc0 += 32) {
      float wv[2][kDirectMaxK / 4];  // W(oc0 + 16 mt + r, tap 4 ks + q)
#pragma unroll
      for (int ks = 0; ks < kDirectMaxK / 4; ++ks)
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const int k = 4 * ks + q;
          wv[mt][ks] = k < K ? a.wt[oc0 + 16 * mt + r + (int64_t)OC * k] : 0.f;
        }
      float bias[2][4];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) bias[mt][i] = a.bias ? a.bias[oc0 + 16 * mt + 4 * q + i] : 0.f;
      // mx[mt][i][nt], mi: channel oc0 + 16 mt + 4 q + i, sample n0 + 4 r + nt
      f32x4 mx[2][4];
      i32x4 mi[2][4];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          mx[mt][i] = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
          mi[mt][i] = i32x4{0, 0, 0, 0};
        }
      f32x4 xv[kDirectMaxK / 4], xn[kDirectMaxK / 4];
      load_x(0, xv);
      for (int sub = 0; sub < nsub; ++sub) {
        if (sub + 1 < nsub) load_x(sub + 1, xn);
        f32x4 acc[2][4];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < kDirectMaxK / 4; ++ks)
          if (ks < nks) {
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
              for (int nt = 0; nt < 4; ++nt)
                acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[mt][ks], xv[ks][nt], acc[mt][nt], 0, 0, 0);
          }
        // as conv_direct_fwd_kernel's epilogue: + bias, then the ReLU
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) {
              float o = acc[mt][nt][i];
              if (a.bias) o = o + bias[mt][i];
              o = relu_f(o);
              if (o > mx[mt][i][nt]) {
                mx[mt][i][nt] = o;
                mi[mt][i][nt] = sub;
              }
            }
#pragma unroll
        for (int ks = 0; ks < kDirectMaxK / 4; ++ks) xv[ks] = xn[ks];
      }
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int64_t o = n0 + 4 * r + d.N * (oc0 + 16 * mt + 4 * q + i + (int64_t)d.OC * pp);
          *reinterpret_cast<f32x4*>(P + o) = mx[mt][i];
          *reinterpret_cast<i32x4*>(pidx + o) = mi[mt][i];
        }
    }
  }
}

// ---------------------------------------------------------------- wgrad
// M = OC, Ng = C*T (+1 ones-column for the bias), contraction index
// k = n + N*q over (sample, output pixel); split over blockIdx.z.
// A(oc, k) = dY[n + N*(oc + OC*q)], B(j, k) = X(n, ic, ih, iw) for
// j = ic + C*t < CT, 1 for j == CT: both contiguous along k within a pixel.
// POOLED: A is the gradient at the conv output of a Conv2D -> ReLU ->
// MaxPool2D stack (windows pool x pool, stride pool, tiling the output),
// formed while loading from the pooled gradient dP, its argmax and the
// pooled output P, as the pool's backward (maxpool_bwd_tiled_vec_kernel,
// ReLU mask from the pooled output) would have written it: conv output
// pixel (oh, ow) in window (oh / pool, ow / pool) at offset s = (oh % pool)
// pool + ow % pool takes (0 + dP) * [P > 0] where the argmax is s, else 0.
// The same values enter the same MFMAs, so the weight and bias gradients
// equal those of the two launches bit for bit, and that gradient (the size
// of the conv output) is never written.
template <class C, bool ALIGNED, bool FAST, bool POOLED = false>
struct WgradStage {
  using OA = kp::Operand<true, C::BM, C::NT, C::KT>;
  using OB = kp::Operand<true, C::BN, C::NT, C::KT>;
  const ConvArgs& a;
  int64_t m0, n0, k_begin, k_end;
  int bic[OB::PER], bkh[OB::PER], bkw[OB::PER];  // row j of each B unit; bic -1: zero, -2: ones
  f32x4 ra[2][OA::REGS], rb[2][OB::REGS];

  __device__ WgradStage(const ConvArgs& a_, int64_t m0_, int64_t n0_, int64_t kb, int64_t ke)
      : a(a_), m0(m0_), n0(n0_), k_begin(kb), k_end(ke) {
    const ConvDims& d = a.d;
    const int64_t CT = d.C * d.KS * d.KS;
#pragma unroll
    for (int p = 0; p < OB::PER; ++p) {
      int r, k;
      bic[p] = -1;
      bkh[p] = bkw[p] = 0;
      if (!OB::origin(p, r, k)) break;
      const int64_t j = n0 + r;
      if (j < CT) {
        const int64_t t = j / d.C;
        bic[p] = (int)(j % d.C);
        bkh[p] = (int)(t % d.KS);
        bkw[p] = (int)(t / d.KS);
      } else if (j == CT && a.has_bias) {
        bic[p] = -2;
      }
    }
  }

  template <int S>
  __device__ __forceinline__ void load(int t) {
    const ConvDims& d = a.d;
    const int64_t k0 = k_begin + (int64_t)t * C::KT;
    if (ALIGNED) {
      // the whole k-tile lies in output pixel q (N % KT == 0), and every
      // tile of the split is full (k_per_split and N*HO*WO are multiples of KT)
      const int N = (int)d.N, HO = (int)d.HO;
      const int q = (int)(k0 / N), nb = (int)(k0 - (int64_t)q * N);
      const int oh = q % HO, ow = q / HO;
      if constexpr (POOLED) {
        typedef int i32x4 __attribute__((ext_vector_type(4)));
        const int pool = a.pool;
        const int s = (oh % pool) * pool + ow % pool;
        const int64_t pbase = nb + d.N * d.OC * ((int64_t)(oh / pool) + a.HP * (int64_t)(ow / pool));
#pragma unroll
        for (int p = 0; p < OA::PER; ++p) {
          int r, k;
          if (!OA::origin(p, r, k)) break;
          f32x4 v{0.f, 0.f, 0.f, 0.f};
          if (FAST || m0 + r < d.OC) {
            const int64_t o = pbase + k + d.N * (m0 + r);
            f32x4 gy = 0.f + *reinterpret_cast<const f32x4*>(a.dY + o);
            const f32x4 yv = *reinterpret_cast<const f32x4*>(a.pout + o);
            const i32x4 mi = *reinterpret_cast<const i32x4*>(a.pidx + o);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              gy[e] *= relu_mask(yv[e]);
              v[e] = mi[e] == s ? gy[e] : 0.f;
            }
          }
          ra[S][p] = v;
        }
      } else {
        OA::template load<FAST>(a.dY + nb + d.N * d.OC * q, d.N, m0, 0, d.OC, C::KT, ra[S]);
      }
      const int ih0 = oh * (int)d.S - (int)d.P, iw0 = ow * (int)d.S - (int)d.P;
#pragma unroll
      for (int p = 0; p < OB::PER; ++p) {
        int r, k;
        if (!OB::origin(p, r, k)) break;
        f32x4 v{0.f, 0.f, 0.f, 0.f};
        if (bic[p] == -2) {
          v = f32x4{1.f, 1.f, 1.f, 1.f};
        } else if (bic[p] >= 0) {
          const int ih = ih0 + bkh[p], iw = iw0 + bkw[p];
          if (ih >= 0 && ih < (int)d.H && iw >= 0 && iw < (int)d.W)
            v = *reinterpret_cast<const f32x4*>(a.src + nb + k +
                                                d.N * (bic[p] + d.C * (ih + d.H * (int64_t)iw)));
        }
        rb[S][p] = v;
      }
    } else {
      // general N: decode (n, q) per element
#pragma unroll
      for (int p = 0; p < OA::PER; ++p) {
        int r, k;
        if (!OA::origin(p, r, k)) break;
        const int64_t oc = m0 + r;
        f32x4 v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t kk = k0 + k + j;
          if (oc < d.OC && kk < k_end) {
            const int64_t n = kk % d.N, q = kk / d.N;
            v[j] = a.dY[n + d.N * (oc + d.OC * q)];
          }
        }
        ra[S][p] = v;
      }
#pragma unroll
      for (int p = 0; p < OB::PER; ++p) {
        int r, k;
        if (!OB::origin(p, r, k)) break;
        f32x4 v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t kk = k0 + k + j;
          if (kk >= k_end || bic[p] == -1) continue;
          if (bic[p] == -2) {
            v[j] = 1.f;
            continue;
          }
          const int64_t n = kk % d.N, q = kk / d.N;
          const int64_t ih = (q % d.HO) * d.S - d.P + bkh[p], iw = (q / d.HO) * d.S - d.P + bkw[p];
          if (ih >= 0 && ih < d.H && iw >= 0 && iw < d.W)
            v[j] = a.src[n + d.N * (bic[p] + d.C * (ih + d.H * iw))];
        }
        rb[S][p] = v;
      }
    }
  }
  template <int S>
  __device__ __forceinline__ void store(float* buf) {
    OA::store(buf, ra[S]);
    OB::store(buf + OA::FLOATS, rb[S]);
  }
};

template <class C, bool ALIGNED, bool POOLED = false>
__global__ void __launch_bounds__(C::NT) conv_wgrad_kernel(ConvArgs a) {
  static_assert(!POOLED || ALIGNED, "the pooled operand needs whole k-tiles within a pixel");
  constexpr int FLOATS = 2 * kp::stage_floats<WgradStage<C, ALIGNED, true, POOLED>>();
  __shared__ __align__(16) float lds[FLOATS];
  static_assert((C::WGK - 1) * C::WGM * C::WGN * C::WM * C::WN * 1024 <= FLOATS,
                "reduce_wgk needs more LDS than the operand buffers");
  const ConvDims& d = a.d;
  const int64_t CT = d.C * d.KS * d.KS, Ng = CT + a.has_bias, Kc = d.N * d.HO * d.WO;
  const int nbm = (int)((d.OC + C::BM - 1) / C::BM);
  // gridDim.x tiles, gridDim.z splits: the tiles of a split (which share its
  // rows of dY) and neighbouring splits go to one XCD
  const int lb = xcd_contiguous((int)(blockIdx.x + gridDim.x * blockIdx.z), (int)(gridDim.x * gridDim.z));
  const int tile = lb % (int)gridDim.x, split = lb / (int)gridDim.x;
  const int64_t m0 = (int64_t)(tile % nbm) * C::BM;
  const int64_t n0 = (int64_t)(tile / nbm) * C::BN;
  const int64_t k_begin = (int64_t)split * a.k_per_split;
  const int64_t k_end = min(Kc, k_begin + a.k_per_split);
  const int ntiles = k_end > k_begin ? (int)((k_end - k_begin + C::KT - 1) / C::KT) : 0;
  f32x16 acc[C::WM][C::WN];
  kp::zero_acc<C>(acc);
  if (ALIGNED && m0 + C::BM <= d.OC) {
    WgradStage<C, ALIGNED, true, POOLED> s(a, m0, n0, k_begin, k_end);
    kp::pipeline<C>(ntiles, lds, s, acc);
  } else {
    WgradStage<C, ALIGNED, false, POOLED> s(a, m0, n0, k_begin, k_end);
    kp::pipeline<C>(ntiles, lds, s, acc);
  }
  kp::reduce_wgk<C>(lds, acc);

  float* P = a.partial + (int64_t)split * d.OC * Ng;
  const bool p_vec = (d.OC & 3) == 0;
  kp::for_each_acc_run<C>(acc, [&](int ml, int nl, const f32x4& v) {
    const int64_t m = m0 + ml, j = n0 + nl;
    if (j >= Ng) return;
    if (p_vec && m + 3 < d.OC) {
      *reinterpret_cast<f32x4*>(P + m + d.OC * j) = v;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (m + e < d.OC) P[(m + e) + d.OC * j] = v[e];
    }
  });
}

// Weight gradient with one output pixel per block (OC = 64, C*k^2 <= 16 CG
// NBW, N % 32 == 0): the block's split of the contraction is exactly the N
// samples of its pixel, so the whole [64, C*k^2] gradient of that pixel is
// one block's tile and every block runs the chip's full MFMA rate for its
// whole life (the 64 x 64 tiles above take C*k^2 / 64 blocks per pixel,
// each a few k-tiles long).  The pixel fixes every tap's input pixel, so
// each thread's gather offsets are computed once and advance by 32 samples
// per k-tile.  Wave (rb, cg): output rows 16 rb .. (oc) and column blocks
// cg NBW .. cg NBW + NBW - 1 (j = c + C (kh + KS kw)) on
// v_mfma_f32_16x16x4f32, lane (q, r) supplying k = 16 s + 4 q + e to MFMA
// (s, e) from float4 LDS reads of rows k-contiguous.  The bias column is the
// sum of the wave's A operands (waves cg = 0).  Partials go to the same
// [pixel][oc + OC*j] layout as conv_wgrad_kernel's splits, for the same
// reduce.
constexpr int PXW_KT = 32;  // samples per k-tile

// Unit u (a float4: 4 samples of one row) of a k-tile -> its row; its 4-sample
// chunk is u & 7.  Rows are 36 floats apart in LDS, conflict-free for the
// fragment reads; the 16 lanes that one ds_write_b128 cycle serves write
// rows r and r + 8 (36 * 8 = 288 = 32 mod 64 banks apart: disjoint halves)
// rather than r and r + 1, whose 32-bank spans overlap by 4.  Global loads
// stay 128-byte runs per 8 lanes.
__device__ __forceinline__ int pxw_row(int u) {
  return ((u >> 7) << 4) | (((u >> 3) & 1) << 3) | ((u >> 4) & 7);
}

// j / dv and j % dv for 0 <= j < 2^20, 1 <= dv: the quotient estimated from
// an approximate float reciprocal (off by at most one, since the product's
// error is below 2^20 * 2^-22) and corrected by the remainder's sign and
// size.  A 32-bit integer division by a runtime divisor is a ~40-instruction
// sequence; the block prologues below decode several per thread.
__device__ __forceinline__ int divmod_small(int j, int dv, float inv, int& rem) {
  int q = (int)((float)j * inv);
  int r = j - q * dv;
  if (r < 0) {
    --q;
    r += dv;
  } else if (r >= dv) {
    ++q;
    r -= dv;
  }
  rem = r;
  return q;
}

template <int CG, int NBW>
__global__ void __launch_bounds__(256 * CG, 1) conv_wgrad_px_kernel(ConvArgs a) {
  constexpr int MB = 4, NT = 64 * MB * CG;
  constexpr int NJ = 16 * CG * NBW;          // B rows j (columns of dW), padded
  static_assert(NJ % 16 == 0, "pxw_row maps 16-row groups");
  constexpr int LD = PXW_KT + 4;             // LDS row stride in floats
  constexpr int AF = 64 * LD, SF = AF + NJ * LD;
  constexpr int AU = 64 * PXW_KT / 4, BU = NJ * PXW_KT / 4;  // float4 units per k-tile
  constexpr int APT = (AU + NT - 1) / NT, BPT = (BU + NT - 1) / NT;
  __shared__ __align__(16) float lds[2 * SF];
  const ConvDims& d = a.d;
  const int N = (int)d.N, C = (int)d.C, KS = (int)d.KS, HO = (int)d.HO;
  const int CT = C * KS * KS;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int q = lane >> 4, r = lane & 15;
  const int rb = wave % MB, cg = wave / MB;
  const int pix = xcd_contiguous((int)blockIdx.x, (int)gridDim.x);
  int oh;
  const int ow = divmod_small(pix, HO, __builtin_amdgcn_rcpf((float)HO), oh);
  // gather offsets (sample 0 of the unit's 4) and LDS slots of this thread's units
  int aoff[APT], boff[BPT];
  const float inv_c = __builtin_amdgcn_rcpf((float)C), inv_ks = __builtin_amdgcn_rcpf((float)KS);
#pragma unroll
  for (int i = 0; i < APT; ++i) {
    const int u = tid + NT * i;
    aoff[i] = u < AU ? 4 * (u & 7) + N * (pxw_row(u) + 64 * pix) : -1;
  }
#pragma unroll
  for (int i = 0; i < BPT; ++i) {
    const int u = tid + NT * i, j = pxw_row(u);
    boff[i] = -2;  // no unit
    if (u < BU) {
      boff[i] = -1;  // zero: padding column or padded input pixel
      if (j < CT) {
        int c, kh;
        const int t = divmod_small(j, C, inv_c, c), kw = divmod_small(t, KS, inv_ks, kh);
        const int ih = oh * (int)d.S - (int)d.P + kh, iw = ow * (int)d.S - (int)d.P + kw;
        if (ih >= 0 && ih < (int)d.H && iw >= 0 && iw < (int)d.W)
          boff[i] = 4 * (u & 7) + N * (c + C * (ih + (int)d.H * iw));
      }
    }
  }
  f32x4 ra[2][APT], rbv[2][BPT];
  auto load = [&](auto slot, int kt) {
    constexpr int S = decltype(slot)::value;
    const int nb = PXW_KT * kt;
#pragma unroll
    for (int i = 0; i < APT; ++i)
      if (aoff[i] >= 0) ra[S][i] = *reinterpret_cast<const f32x4*>(a.dY + aoff[i] + nb);
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
      if (boff[i] >= 0) v = *reinterpret_cast<const f32x4*>(a.src + boff[i] + nb);
      rbv[S][i] = v;
    }
  };
  auto store = [&](auto slot) {
    constexpr int S = decltype(slot)::value;
    float* buf = lds + S * SF;
#pragma unroll
    for (int i = 0; i < APT; ++i) {
      const int u = tid + NT * i;
      if (u < AU) *reinterpret_cast<f32x4*>(buf + pxw_row(u) * LD + 4 * (u & 7)) = ra[S][i];
    }
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      const int u = tid + NT * i;
      if (u < BU) *reinterpret_cast<f32x4*>(buf + AF + pxw_row(u) * LD + 4 * (u & 7)) = rbv[S][i];
    }
  };
  f32x4 acc[NBW];
#pragma unroll
  for (int c = 0; c < NBW; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  float bsum = 0.f;
  auto compute = [&](auto slot) {
    constexpr int S = decltype(slot)::value;
    const float* As = lds + S * SF;
    const float* Bs = As + AF;
#pragma unroll
    for (int s = 0; s < PXW_KT / 16; ++s) {
      const f32x4 av = *reinterpret_cast<const f32x4*>(As + (16 * rb + r) * LD + 16 * s + 4 * q);
      f32x4 bv[NBW];
#pragma unroll
      for (int c = 0; c < NBW; ++c)
        bv[c] = *reinterpret_cast<const f32x4*>(Bs + (16 * (cg * NBW + c) + r) * LD + 16 * s + 4 * q);
      // raised issue priority while this wave's MFMAs are queued (the other
      // wave on the SIMD is then more often the one staging operands)
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int c = 0; c < NBW; ++c) acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[e], bv[c][e], acc[c], 0, 0, 0);
      __builtin_amdgcn_s_setprio(0);
      if (cg == 0) bsum += (av[0] + av[1]) + (av[2] + av[3]);
    }
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  const int nkt = N / PXW_KT;
  load(S0{}, 0);
  if (nkt > 1) load(S1{}, 1);
  store(S0{});
  __syncthreads();
  // tile kt sits in LDS buffer kt & 1; the registers of slot kt & 1 are
  // refilled with tile kt + 2 once tile kt has been stored
  for (int kt = 0; kt < nkt; kt += 2) {
    if (kt + 2 < nkt) load(S0{}, kt + 2);
    compute(S0{});
    if (kt + 1 < nkt) store(S1{});
    __syncthreads();
    if (kt + 1 >= nkt) break;
    if (kt + 3 < nkt) load(S1{}, kt + 3);
    compute(S1{});
    if (kt + 2 < nkt) store(S0{});
    __syncthreads();
  }
  const int64_t OC = d.OC;
  float* P = a.partial + (int64_t)pix * OC * (CT + a.has_bias);
#pragma unroll
  for (int c = 0; c < NBW; ++c) {
    const int j = 16 * (cg * NBW + c) + r;
    if (j < CT) *reinterpret_cast<f32x4*>(P + 16 * rb + 4 * q + OC * j) = acc[c];
  }
  if (cg == 0 && a.has_bias) {
    bsum += __shfl_xor(bsum, 16, 64);
    bsum += __shfl_xor(bsum, 32, 64);
    if (q == 0) P[16 * rb + r + OC * CT] = bsum;
  }
}

// Shapes conv_wgrad_px_kernel<CG, NBW> serves.
bool wgrad_px_serves(const ConvArgs& a, int CG, int NBW) {
  const ConvDims& d = a.d;
  return a.pool == 0 && a.aligned && d.OC == 64 && d.N % PXW_KT == 0 && d.N >= 4 * PXW_KT &&
         d.C * d.KS * d.KS <= 16 * CG * NBW && d.HO * d.WO <= 1024 &&
         d.N * d.C * d.H * d.W < ((int64_t)1 << 31) && d.N * d.OC * d.HO * d.WO < ((int64_t)1 << 31);
}

// gW[oc + OC*j] = sum_z partial[z][oc + OC*j]; the ones-column goes to gb.
// 64 consecutive outputs per block (coalesced along e); the RW waves of a
// block each sum one contiguous chunk of z in ascending order, and the chunk
// sums are added in ascending order: a fixed summation order for any launch.
constexpr int WGRAD_RW = 16;
// With Wr set, the same launch also writes the input-gradient pass's copy of
// W as [OC*T, C]: Wr[k' + OC*T*ic] = W[oc + OC*(ic + C*t)], k' = oc + OC*t,
// T = CT / C.  W does not change during the backward, so the copy needs no
// launch of its own (a separate one cost ~4.6 us for 18 K floats at config
// 3's conv2).
__global__ void __launch_bounds__(64 * WGRAD_RW) conv_wgrad_reduce_kernel(
    const float* __restrict__ partial, int splits, int64_t OC, int64_t CT, int has_bias,
    float* __restrict__ gW, float* __restrict__ gb, const float* __restrict__ W,
    float* __restrict__ Wr, int64_t C) {
  __shared__ float part[WGRAD_RW][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t Ng = CT + has_bias, total = OC * Ng;
  const int64_t e = (int64_t)blockIdx.x * 64 + lane;
  const int per = (splits + WGRAD_RW - 1) / WGRAD_RW;
  const int z0 = w * per, z1 = min(splits, z0 + per);
  float s = 0.f;
  if (e < total) {
#pragma unroll 8
    for (int z = z0; z < z1; ++z) s += partial[(int64_t)z * total + e];
  }
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
  if (Wr) {
    const int64_t T = CT / C, Kp = OC * T, n = OC * CT;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
      const int64_t oc = i % OC, ic = (i / OC) % C, t = i / (OC * C);
      Wr[(oc + OC * t) + Kp * ic] = W[i];
    }
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

// Per-pixel GEMM (M = N along the batch, Ng = OC or C channels) launch.
// `gathered`: elements of the tensor A gathers from (the table holds 32-bit
// offsets into it).
template <bool DGRAD>
void launch_pixel(const ConvArgs& a, int64_t Ng, int64_t K, int64_t pixels, int64_t gathered,
                  hipStream_t st) {
  auto go = [&](auto cfg) {
    using Cfg = decltype(cfg);
    const int64_t kpad = (K + Cfg::KT - 1) / Cfg::KT * Cfg::KT;
    const bool tbl = kpad <= KTBL && gathered < ((int64_t)1 << 31);
    const int64_t tiles = ((a.d.N + Cfg::BM - 1) / Cfg::BM) * ((Ng + Cfg::BN - 1) / Cfg::BN);
    // algorithmic flops: 2 * N * (output pixels) * OC * C * KS^2 in both directions
    const ConvDims& d = a.d;
    TimingRec* rec = timing_slot(2.0 * d.N * d.HO * d.WO * d.OC * d.C * d.KS * d.KS);
    if (rec) (void)hipEventRecord(rec->start, st);
    const auto kern = tbl ? &conv_pixel_kernel<Cfg, DGRAD, true> : &conv_pixel_kernel<Cfg, DGRAD, false>;
    hipLaunchKernelGGL(kern, dim3((unsigned)tiles, (unsigned)pixels), dim3(Cfg::NT), 0, st, a);
    if (rec) (void)hipEventRecord(rec->stop, st);
  };
  // shapes measured fastest on the config-3 layers (N = 256)
  if (Ng <= 32) {
    if (DGRAD) go(kp::Cfg<4, 1, 1, 1, 16, 2>{});  // 128 x 32, k-tile split over 2 wave groups
    else if (a.d.N >= 256) go(kp::Cfg<8, 1, 1, 1>{});  // 256 x 32
    else go(kp::Cfg<4, 1, 1, 1>{});                // 128 x 32
  } else if (Ng <= 64) {
    go(kp::Cfg<4, 2, 1, 1>{});                     // 128 x 64, 8 waves
  } else {
    go(kp::Cfg<2, 2, 2, 2>{});                     // 128 x 128
  }
}

// Weight-gradient launch for an OC x Ng tile grid: split-K partials, then a
// fixed-order sum into gW / gb.  Small tiles split each k-tile over WGK wave
// groups so a block has 4 or 8 waves.
// W and Wr: see conv_wgrad_reduce_kernel (both null: no relayout).
int launch_wgrad(ConvArgs a, float* gW, float* gb, const float* W, float* Wr, hipStream_t st,
                 const char* who) {
  const ConvDims& d = a.d;
  const int64_t CT = d.C * d.KS * d.KS, Ng = CT + a.has_bias, Kc = d.N * d.HO * d.WO;
  // the fixed-order sum of the splits' partials (and W's relayout)
  auto reduce = [&](int64_t splits, int status) -> int {
    if (status == CNHIP_OK) {
      HbmTimer timer("conv_wgrad_reduce_kernel",
                     4.0 * (double)(splits + 1) * d.OC * Ng + (Wr ? 8.0 * (double)d.OC * CT : 0.0), st);
      hipLaunchKernelGGL(conv_wgrad_reduce_kernel, dim3((unsigned)((d.OC * Ng + 63) / 64)),
                         dim3(64 * WGRAD_RW), 0, st, a.partial, (int)splits, d.OC, CT, a.has_bias,
                         gW, gb, W, Wr, d.C);
      status = check_launch(who);
    }
    return status;
  };
  if (wgrad_px_serves(a, 2, 9)) {
    // one output pixel per block: its N samples are the block's split
    const int64_t splits = d.HO * d.WO;
    void* ws = nullptr;
    CNHIP_TRY(scratch(st, kScratchLayer, (size_t)splits * d.OC * Ng * sizeof(float), &ws, who));
    a.partial = static_cast<float*>(ws);
    TimingRec* rec = timing_slot(2.0 * Kc * d.OC * CT);
    if (rec) (void)hipEventRecord(rec->start, st);
    hipLaunchKernelGGL((conv_wgrad_px_kernel<2, 9>), dim3((unsigned)splits), dim3(512), 0, st, a);
    const int status = check_launch(who);
    if (rec) (void)hipEventRecord(rec->stop, st);
    return reduce(splits, status);
  }
  // target: blocks to aim for with split-K (fewer, longer blocks cut the
  // partial traffic; more hide latency), measured per tile shape
  auto go = [&](auto cfg, int64_t target) -> int {
    using Cfg = decltype(cfg);
    a.aligned = a.aligned && d.N % Cfg::KT == 0;
    const int64_t tiles = ((d.OC + Cfg::BM - 1) / Cfg::BM) * ((Ng + Cfg::BN - 1) / Cfg::BN);
    int64_t splits = std::max<int64_t>(1, (target + tiles - 1) / tiles);
    splits = std::min<int64_t>(splits, std::max<int64_t>(1, Kc / (8 * Cfg::KT)));
    int64_t kps = (Kc + splits - 1) / splits;
    kps = (kps + Cfg::KT - 1) / Cfg::KT * Cfg::KT;
    splits = (Kc + kps - 1) / kps;
    a.k_per_split = kps;
    void* ws = nullptr;
    CNHIP_TRY(scratch(st, kScratchLayer, (size_t)splits * d.OC * Ng * sizeof(float), &ws, who));
    a.partial = static_cast<float*>(ws);
    TimingRec* rec = timing_slot(2.0 * Kc * d.OC * CT);
    if (rec) (void)hipEventRecord(rec->start, st);
    CNHIP_REQUIRE(a.pool == 0 || a.aligned, "%s: the pooled weight gradient needs N %% %d == 0 and 16-byte "
                  "aligned tensors", who, Cfg::KT);
    const auto kern = a.pool > 0 ? &conv_wgrad_kernel<Cfg, true, true>
                      : a.aligned ? &conv_wgrad_kernel<Cfg, true> : &conv_wgrad_kernel<Cfg, false>;
    hipLaunchKernelGGL(kern, dim3((unsigned)tiles, 1, (unsigned)splits), dim3(Cfg::NT), 0, st, a);
    const int status = check_launch(who);
    if (rec) (void)hipEventRecord(rec->stop, st);
    return reduce(splits, status);
  };
  const int bm = d.OC <= 32 ? 32 : d.OC <= 64 ? 64 : 128;
  const int bn = Ng <= 32 ? 32 : Ng <= 64 ? 64 : 128;
  if (bm == 32) {
    if (bn == 32) return go(kp::Cfg<1, 1, 1, 1, 16, 4>{}, 512);
    if (bn == 64) return go(kp::Cfg<1, 2, 1, 1, 16, 2>{}, 512);
    return go(kp::Cfg<1, 4, 1, 1, 16, 1>{}, 512);
  }
  if (bm == 64) {
    if (bn == 32) return go(kp::Cfg<2, 1, 1, 1, 16, 2>{}, 512);
    return go(kp::Cfg<2, 2, 1, 1, 16, 2>{}, 2048);  // 64 x 64, 8 waves
  }
  if (bn == 32) return go(kp::Cfg<4, 1, 1, 1, 16, 1>{}, 512);
  if (bn == 64) return go(kp::Cfg<2, 2, 2, 1, 16, 1>{}, 512);
  return go(kp::Cfg<2, 2, 2, 2, 16, 1>{}, 512);
}

}  // namespace
}  // namespace cnhip

using cnhip::as_stream;

namespace {

int conv_forward(const float* X, const float* W, const float* b, float* Y, int64_t N, int64_t C,
                 int64_t H, int64_t Wd, int64_t OC, int64_t KS, int64_t S, int64_t P, int relu,
                 cnhip_stream_t stream, const char* who) {
  const cnhip::ConvDims d = cnhip::make_dims(N, C, H, Wd, OC, KS, S, P);
  CNHIP_TRY(cnhip::check_dims(d, who));
  CNHIP_REQUIRE(X && W && Y, "%s: NULL pointer", who);
  cnhip::ConvArgs a{};
  a.d = d; a.src = X; a.wt = W; a.bias = b; a.out = Y; a.relu = relu;
  a.out_vec = (N % 4 == 0) && cnhip::aligned16(Y);
  a.src_vec = (N % 4 == 0) && cnhip::aligned16(X);
  a.wt_vec = (OC % 4 == 0) && cnhip::aligned16(W);
  if (C * KS * KS <= cnhip::kDirectMaxK && OC % 32 == 0 && N % 64 == 0 && a.out_vec && a.src_vec &&
      (N + 255) / 256 <= 65535 && N * C * H * Wd < ((int64_t)1 << 31)) {
    // short contraction: bound by writing Y (X read once from HBM, then from cache)
    cnhip::HbmTimer timer("conv_direct_fwd_kernel",
                          4.0 * ((double)N * C * H * Wd + (double)N * OC * d.HO * d.WO + (double)OC * C * KS * KS),
                          as_stream(stream));
    // 2 blocks per CU over the 256 CUs: an even share of pixels each
    const int64_t nb = (N + 255) / 256, px = std::min<int64_t>(d.HO * d.WO, std::max<int64_t>(1, 512 / nb));
    hipLaunchKernelGGL(cnhip::conv_direct_fwd_kernel, dim3((unsigned)px, (unsigned)nb), dim3(256), 0,
                       as_stream(stream), a);
    return cnhip::check_launch(who);
  }
  cnhip::launch_pixel<false>(a, OC, C * KS * KS, d.HO * d.WO, N * C * H * Wd, as_stream(stream));
  return cnhip::check_launch(who);
}

}  // namespace

extern "C" {

int cnhip_conv2d_forward(const float* X, const float* W, const float* b, float* Y, int64_t N,
                         int64_t C, int64_t H, int64_t Wd, int64_t OC, int64_t KS, int64_t S,
                         int64_t P, cnhip_stream_t stream) {
  return conv_forward(X, W, b, Y, N, C, H, Wd, OC, KS, S, P, 0, stream, "cnhip_conv2d_forward");
}

int cnhip_conv2d_forward_relu(const float* X, const float* W, const float* b, float* Y, int64_t N,
                              int64_t C, int64_t H, int64_t Wd, int64_t OC, int64_t KS, int64_t S,
                              int64_t P, cnhip_stream_t stream) {
  return conv_forward(X, W, b, Y, N, C, H, Wd, OC, KS, S, P, 1, stream,
                      "cnhip_conv2d_forward_relu");
}

int cnhip_conv2d_forward_relu_maxpool(const float* X, const float* W, const float* b, float* Yp,
                                      int32_t* idx, int64_t N, int64_t C, int64_t H, int64_t Wd,
                                      int64_t OC, int64_t KS, int64_t S, int64_t P, int64_t pool,
                                      int64_t pool_stride, cnhip_stream_t stream) {
  const char* who = "cnhip_conv2d_forward_relu_maxpool";
  const cnhip::ConvDims d = cnhip::make_dims(N, C, H, Wd, OC, KS, S, P);
  CNHIP_TRY(cnhip::check_dims(d, who));
  CNHIP_REQUIRE(X && W && Yp && idx, "%s: NULL pointer", who);
  if (pool_stride <= 0) pool_stride = pool;  // max_pool2d.cpp:25-28
  CNHIP_REQUIRE(pool > 0 && pool <= d.HO && pool <= d.WO, "%s: pool %lld does not fit the %lldx%lld conv output",
                who, (long long)pool, (long long)d.HO, (long long)d.WO);
  hipStream_t st = as_stream(stream);
  const int64_t HP = (d.HO - pool) / pool_stride + 1, WP = (d.WO - pool) / pool_stride + 1;
  cnhip::ConvArgs a{};
  a.d = d; a.src = X; a.wt = W; a.bias = b; a.relu = 1;
  a.src_vec = (N % 4 == 0) && cnhip::aligned16(X);
  if (C * KS * KS <= cnhip::kDirectMaxK && OC % 32 == 0 && N % 64 == 0 && a.src_vec && cnhip::aligned16(Yp) &&
      cnhip::aligned16(idx) && pool_stride == pool && pool <= cnhip::kPoolMaxFused && HP * pool == d.HO &&
      WP * pool == d.WO && (N + 255) / 256 <= 65535 && N * C * H * Wd < ((int64_t)1 << 31) &&
      N * OC * HP * WP < ((int64_t)1 << 31)) {
    // X read once from HBM; the pooled output and the int32 argmax written
    cnhip::HbmTimer timer("conv_direct_pool_fwd_kernel",
                          4.0 * ((double)N * C * H * Wd + (double)OC * C * KS * KS) + 8.0 * (double)N * OC * HP * WP,
                          st);
    const int64_t nb = (N + 255) / 256, px = std::min<int64_t>(HP * WP, std::max<int64_t>(1, 512 / nb));
    hipLaunchKernelGGL(cnhip::conv_direct_pool_fwd_kernel, dim3((unsigned)px, (unsigned)nb), dim3(256), 0, st, a,
                       (int)pool, Yp, idx);
    return cnhip::check_launch(who);
  }
  // any other shape: the conv + ReLU output in a workspace, then the pool
  void* ws = nullptr;
  CNHIP_TRY(cnhip::scratch(st, cnhip::kScratchLayer, (size_t)(N * OC * d.HO * d.WO) * sizeof(float), &ws, who));
  float* Y = static_cast<float*>(ws);
  CNHIP_TRY(conv_forward(X, W, b, Y, N, C, H, Wd, OC, KS, S, P, 1, stream, who));
  return cnhip_maxpool2d_forward(Y, Yp, idx, N, OC, d.HO, d.WO, pool, pool_stride, stream);
}

int cnhip_conv2d_backward_maxpool_relu_fits(int64_t N, int64_t C, int64_t H, int64_t Wd, int64_t OC, int64_t KS,
                                            int64_t S, int64_t P, int64_t pool, int64_t pool_stride) {
  const cnhip::ConvDims d = cnhip::make_dims(N, C, H, Wd, OC, KS, S, P);
  if (pool_stride <= 0) pool_stride = pool;
  return N > 0 && C > 0 && H > 0 && Wd > 0 && OC > 0 && KS > 0 && S > 0 && P >= 0 && d.HO > 0 && d.WO > 0 &&
                 d.HO * d.WO <= 65535 && pool > 0 && pool_stride == pool && d.HO % pool == 0 && d.WO % pool == 0 &&
                 N % 64 == 0 && N * OC * d.HO * d.WO < ((int64_t)1 << 31)
             ? 1
             : 0;
}

int cnhip_conv2d_backward_maxpool_relu(const float* X, const float* dP, const int32_t* idx, const float* Pout,
                                       float* gW, float* gb, int64_t N, int64_t C, int64_t H, int64_t Wd,
                                       int64_t OC, int64_t KS, int64_t S, int64_t P, int64_t pool,
                                       int64_t pool_stride, cnhip_stream_t stream) {
  const char* who = "cnhip_conv2d_backward_maxpool_relu";
  const cnhip::ConvDims d = cnhip::make_dims(N, C, H, Wd, OC, KS, S, P);
  CNHIP_TRY(cnhip::check_dims(d, who));
  CNHIP_REQUIRE(X && dP && idx && Pout && gW, "%s: NULL pointer", who);
  if (pool_stride <= 0) pool_stride = pool;  // max_pool2d.cpp:25-28
  CNHIP_REQUIRE(cnhip_conv2d_backward_maxpool_relu_fits(N, C, H, Wd, OC, KS, S, P, pool, pool_stride),
                "%s: needs pool windows that tile the %lldx%lld conv output (stride == pool), N %% 64 == 0 and "
                "fewer than 2^31 conv outputs (N=%lld OC=%lld pool=%lld stride=%lld)",
                who, (long long)d.HO, (long long)d.WO, (long long)N, (long long)OC, (long long)pool,
                (long long)pool_stride);
  CNHIP_REQUIRE(cnhip::aligned16(X) && cnhip::aligned16(dP) && cnhip::aligned16(idx) && cnhip::aligned16(Pout),
                "%s: X, dP, idx and the pooled output must be 16-byte aligned", who);
  cnhip::ConvArgs a{};
  a.d = d; a.src = X; a.dY = dP;
  a.has_bias = gb ? 1 : 0;
  a.aligned = 1;
  a.pidx = idx; a.pout = Pout; a.pool = (int)pool; a.HP = d.HO / pool;
  return cnhip::launch_wgrad(a, gW, gb, nullptr, nullptr, as_stream(stream), who);
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
  a.d = d; a.src = X; a.dY = dY;
  a.has_bias = gb ? 1 : 0;
  a.aligned = cnhip::aligned16(X) && cnhip::aligned16(dY);  // N % KT is checked per tile shape
  // W relaid out as [OC*T, C] for the input gradient, written by the weight
  // gradient's reduce launch into the GEMM scratch slot (the wgrad partials
  // hold the layer slot; nothing on this path runs a GEMM)
  float* Wr = nullptr;
  if (dX) {
    void* ws = nullptr;
    CNHIP_TRY(cnhip::scratch(st, cnhip::kScratchGemm, (size_t)OC * CT * sizeof(float), &ws, who));
    Wr = static_cast<float*>(ws);
  }
  CNHIP_TRY(cnhip::launch_wgrad(a, gW, gb, W, Wr, st, who));

  // ---- input grad: per-input-pixel GEMMs over the relaid-out W
  if (dX) {
    cnhip::ConvArgs b{};
    b.d = d; b.src = dY; b.wt = Wr; b.out = dX;
    b.out_vec = (N % 4 == 0) && cnhip::aligned16(dX);
    b.src_vec = (N % 4 == 0) && cnhip::aligned16(dY);
    b.wt_vec = (OC * T) % 4 == 0;  // Wr is a scratch buffer: 256-byte aligned
    cnhip::launch_pixel<true>(b, C, OC * T, H * Wd, N * OC * d.HO * d.WO, st);
    CNHIP_TRY(cnhip::check_launch(who));
  }
  return CNHIP_OK;
}

}  // extern "C"
