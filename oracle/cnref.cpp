// CPU oracle for the CppNet "cpu-eigen" semantics — TEST INFRASTRUCTURE ONLY
// (loaded by tests/, smoke() and bench.py's cpu_baseline leg; never by the
// product).  See cnref.h for conventions.  Reference paths are relative to
// the LoqmanSamani/CppNet tree.
#include "cnref.h"
#include "cnref_fn.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

namespace cnref_detail {
int acc_double = 0;
}

namespace {
int g_threads = 1;
int& g_acc_double = cnref_detail::acc_double;
int g_order = 0;
int g_cpu_loops = 0;

// dst[r + R c] = trans ? src[c + ld r] : src[r + ld c], in 64 x 64 tiles.
void copy_tiles(float* dst, int64_t R, int64_t Cn, const float* src, int64_t ld, bool trans) {
  constexpr int64_t T = 64;
  const int64_t tr = (R + T - 1) / T, tc = (Cn + T - 1) / T;
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int64_t t = 0; t < tr * tc; ++t) {
    const int64_t r0 = (t % tr) * T, c0 = (t / tr) * T;
    const int64_t r1 = std::min(R, r0 + T), c1 = std::min(Cn, c0 + T);
    if (trans) {
      for (int64_t r = r0; r < r1; ++r)
        for (int64_t c = c0; c < c1; ++c) dst[r + R * c] = src[c + ld * r];
    } else {
      for (int64_t c = c0; c < c1; ++c)
        for (int64_t r = r0; r < r1; ++r) dst[r + R * c] = src[r + ld * c];
    }
  }
}

// acc[m + M n] += sum_k Am[m + M k] * Bk[k + K n] in the accumulator type
// T, each element's products added in the order ORD:
//   0  ascending k (the restatement's order);
//   1  descending k;
//   2  32-wide chunks of k, each summed from zero in ascending k, the chunk
//      sums added in ascending order (the shape of a tiled accumulation);
//   3  within each k-panel of KB, P = 8 strided partial sums (k mod 8, each
//      ascending), combined by a pairwise tree and added panel after panel
//      (the shape of lane-parallel partial sums reduced across lanes).
// An MR x 4 tile of acc is held in registers across a k-panel of KB
// (MR = 64 bytes of T).
constexpr int KP = 8;  // partial sums of order 3
// ((q0 + q1) + (q2 + q3)) + ((q4 + q5) + (q6 + q7))
template <class T>
T tree8(const T* q) {
  return ((q[0] + q[1]) + (q[2] + q[3])) + ((q[4] + q[5]) + (q[6] + q[7]));
}

template <class T, int ORD>
void gemm_panels(int64_t M, int64_t N, int64_t K, const float* Am, const float* Bk, T* acc) {
  constexpr int64_t KB = 256, NB = 4, MR = 64 / sizeof(T), KC = 32;
  const int64_t nblocks = (N + NB - 1) / NB;
  const int64_t npanels = (K + KB - 1) / KB;
  for (int64_t pi = 0; pi < npanels; ++pi) {
    const int64_t k0 = (ORD == 1 ? npanels - 1 - pi : pi) * KB;
    const int64_t k1 = std::min(K, k0 + KB);
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t nb = 0; nb < nblocks; ++nb) {
      const int64_t n0 = nb * NB, nn = std::min(NB, N - n0);
      const float* bcol[NB];
      for (int64_t j = 0; j < NB; ++j) bcol[j] = Bk + K * (n0 + std::min(j, nn - 1));
      int64_t m0 = 0;
      if (nn == NB) {
        for (; m0 + MR <= M; m0 += MR) {
          T c[NB][MR];
          for (int64_t j = 0; j < NB; ++j)
            for (int64_t i = 0; i < MR; ++i) c[j][i] = acc[m0 + i + M * (n0 + j)];
          if (ORD == 3) {
            T part[KP][NB][MR];
            for (int p = 0; p < KP; ++p)
              for (int64_t j = 0; j < NB; ++j)
                for (int64_t i = 0; i < MR; ++i) part[p][j][i] = 0;
            for (int64_t k = k0; k < k1; ++k) {
              T (&dst)[NB][MR] = part[(k - k0) % KP];
              const float* a = Am + m0 + M * k;
              T av[MR];
              for (int64_t i = 0; i < MR; ++i) av[i] = a[i];
              for (int64_t j = 0; j < NB; ++j) {
                const T b = bcol[j][k];
                for (int64_t i = 0; i < MR; ++i) dst[j][i] += av[i] * b;
              }
            }
            for (int64_t j = 0; j < NB; ++j)
              for (int64_t i = 0; i < MR; ++i) {
                T q[KP];
                for (int p = 0; p < KP; ++p) q[p] = part[p][j][i];
                c[j][i] += tree8(q);
              }
          }
          for (int64_t kc = k0; ORD != 3 && kc < k1; kc += KC) {
            const int64_t kc1 = std::min(k1, kc + KC);
            T part[NB][MR];
            for (int64_t j = 0; j < NB; ++j)
              for (int64_t i = 0; i < MR; ++i) part[j][i] = 0;
            T (&dst)[NB][MR] = ORD == 2 ? part : c;
            for (int64_t kk = kc; kk < kc1; ++kk) {
              const int64_t k = ORD == 1 ? (k0 + k1 - 1) - kk : kk;
              const float* a = Am + m0 + M * k;
              T av[MR];
              for (int64_t i = 0; i < MR; ++i) av[i] = a[i];
              for (int64_t j = 0; j < NB; ++j) {
                const T b = bcol[j][k];
                for (int64_t i = 0; i < MR; ++i) dst[j][i] += av[i] * b;
              }
            }
            if (ORD == 2)
              for (int64_t j = 0; j < NB; ++j)
                for (int64_t i = 0; i < MR; ++i) c[j][i] += part[j][i];
          }
          for (int64_t j = 0; j < NB; ++j)
            for (int64_t i = 0; i < MR; ++i) acc[m0 + i + M * (n0 + j)] = c[j][i];
        }
      }
      // rows past the last full tile, and the last partial column block
      for (int64_t j = 0; j < nn; ++j) {
        T* cc = acc + M * (n0 + j);
        for (int64_t m = m0; m < M; ++m) {
          T cm = cc[m];
          if (ORD == 3) {
            T q[KP] = {};
            for (int64_t k = k0; k < k1; ++k) q[(k - k0) % KP] += (T)Am[m + M * k] * (T)bcol[j][k];
            cm += tree8(q);
          }
          for (int64_t kc = k0; ORD != 3 && kc < k1; kc += KC) {
            const int64_t kc1 = std::min(k1, kc + KC);
            T part = 0;
            T& dst = ORD == 2 ? part : cm;
            for (int64_t kk = kc; kk < kc1; ++kk) {
              const int64_t k = ORD == 1 ? (k0 + k1 - 1) - kk : kk;
              dst += (T)Am[m + M * k] * (T)bcol[j][k];
            }
            if (ORD == 2) cm += part;
          }
          cc[m] = cm;
        }
      }
    }
  }
}
}  // namespace

namespace {
// Sum of term(i) over i in [0, n), in the evaluation order the tests select
// (cnref_set_sum_order / cnref_set_accumulate_double; default: ascending i
// in fp32, each addition rounded once).
template <class F>
float osum(int64_t n, F term) {
  if (g_acc_double) {
    double s = 0.0;
    for (int64_t i = 0; i < n; ++i) s += (double)term(i);
    return (float)s;
  }
  float s = 0.0f;
  if (g_order == 1) {
    for (int64_t i = n - 1; i >= 0; --i) s += term(i);
  } else if (g_order == 2) {
    for (int64_t c = 0; c < n; c += 32) {
      float p = 0.0f;
      for (int64_t i = c; i < std::min(n, c + 32); ++i) p += term(i);
      s += p;
    }
  } else if (g_order == 3) {
    float q[KP] = {};
    for (int64_t i = 0; i < n; ++i) q[i % KP] += term(i);
    s = tree8(q);
  } else {
    for (int64_t i = 0; i < n; ++i) s += term(i);
  }
  return s;
}

// out[j] = sum over i in [0, n) of the contributions add(i, acc) makes to
// acc[j] (j < width), in the selected order, like osum.
template <class T, class F>
void osum_into_t(int64_t n, int64_t width, float* out, F add) {
  std::vector<T> acc((size_t)width, T(0)), part((size_t)width);
  if (g_order == 1 && !g_acc_double) {
    for (int64_t i = n - 1; i >= 0; --i) add(i, acc.data());
  } else if (g_order == 2 && !g_acc_double) {
    for (int64_t c = 0; c < n; c += 32) {
      std::fill(part.begin(), part.end(), T(0));
      for (int64_t i = c; i < std::min(n, c + 32); ++i) add(i, part.data());
      for (int64_t j = 0; j < width; ++j) acc[(size_t)j] += part[(size_t)j];
    }
  } else if (g_order == 3 && !g_acc_double) {
    std::vector<T> parts((size_t)(KP * width), T(0));
    for (int64_t i = 0; i < n; ++i) add(i, parts.data() + (size_t)((i % KP) * width));
    for (int64_t j = 0; j < width; ++j) {
      T q[KP];
      for (int p = 0; p < KP; ++p) q[p] = parts[(size_t)(p * width + j)];
      acc[(size_t)j] = tree8(q);
    }
  } else {
    for (int64_t i = 0; i < n; ++i) add(i, acc.data());
  }
  for (int64_t j = 0; j < width; ++j) out[j] = (float)acc[(size_t)j];
}
template <class F>
void osum_into(int64_t n, int64_t width, float* out, F add) {
  if (g_acc_double)
    osum_into_t<double>(n, width, out, add);
  else
    osum_into_t<float>(n, width, out, add);
}
}  // namespace

extern "C" {

static float* g_trace[5] = {};
void cnref_set_trace(int slot, float* buf) {
  if (slot >= 0 && slot < 5) g_trace[slot] = buf;
}
float* cnref_trace(int slot) { return slot >= 0 && slot < 5 ? g_trace[slot] : nullptr; }

void cnref_set_threads(int n) { g_threads = n < 1 ? 1 : n; }
int cnref_get_threads(void) { return g_threads; }
void cnref_set_accumulate_double(int on) { g_acc_double = on != 0; }
void cnref_set_sum_order(int order) { g_order = order >= 0 && order <= 3 ? order : 0; }
void cnref_set_cpu_loops(int on) { g_cpu_loops = on != 0; }
int cnref_get_cpu_loops(void) { return g_cpu_loops; }

// ---------------------------------------------------------------------------
// GEMM.  op(A) is first materialised M-contiguous and op(B) K-contiguous;
// each column n of the product is then accumulated as a sequence of axpys in
// ascending k, so element (m,n) is the fp32 sum  ((0 + a0 b0) + a1 b1) + ...
// This is the contraction Eigen performs for X.contract(W) in
// Linear::forward_eigen (linear.cpp:224) and backward_eigen (346-357), up to
// Eigen's blocking of the k loop.
void cnref_gemm_f32(int ta, int tb, int64_t M, int64_t N, int64_t K, float alpha, const float* A,
                    int64_t lda, const float* B, int64_t ldb, float beta, float* C, int64_t ldc,
                    const float* bias, int epi) {
  if (M <= 0 || N <= 0) return;
  std::vector<float> Am((size_t)M * (size_t)std::max<int64_t>(K, 1));
  std::vector<float> Bk((size_t)std::max<int64_t>(K, 1) * (size_t)N);
  copy_tiles(Am.data(), M, K, A, lda, ta != 0);   // Am[m + M k] = op(A)(m, k)
  copy_tiles(Bk.data(), K, N, B, ldb, tb != 0);   // Bk[k + K n] = op(B)(k, n)

  // Blocked for the cache without changing any element's arithmetic: a
  // k-panel of KB is applied to a 4-column x MB-row block of the product
  // (4 accumulator columns stay in L1 and each A value is loaded once for
  // all four), panel after panel, so element (m, n) still receives its
  // products in ascending k, one rounding per multiply and per add.
  std::vector<float> acc((size_t)M * (size_t)N, 0.f);
  if (g_acc_double) {
    // Variant used only to measure how far a trajectory moves under a
    // different (more accurate) summation: products and sums in double,
    // one rounding to float per element.
    std::vector<double> accd((size_t)M * (size_t)N, 0.0);
    gemm_panels<double, 0>(M, N, K, Am.data(), Bk.data(), accd.data());
    for (size_t i = 0; i < acc.size(); ++i) acc[i] = (float)accd[i];
  } else if (g_order == 1) {
    gemm_panels<float, 1>(M, N, K, Am.data(), Bk.data(), acc.data());
  } else if (g_order == 2) {
    gemm_panels<float, 2>(M, N, K, Am.data(), Bk.data(), acc.data());
  } else if (g_order == 3) {
    gemm_panels<float, 3>(M, N, K, Am.data(), Bk.data(), acc.data());
  } else {
    gemm_panels<float, 0>(M, N, K, Am.data(), Bk.data(), acc.data());
  }
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int64_t n = 0; n < N; ++n)
    for (int64_t m = 0; m < M; ++m) {
      float v = alpha * acc[m + M * n];
      if (beta != 0.f) v += beta * C[m + ldc * n];
      if (bias) v += bias[n];
      if (epi == 1) v = std::max(v, 0.f);
      C[m + ldc * n] = v;
    }
}

// Linear::forward_eigen (linear.cpp:218-234): output = X.contract(W) then
// + bias broadcast along the batch.
void cnref_linear_forward(const float* X, const float* W, const float* b, float* Y, int64_t B,
                          int64_t I, int64_t O) {
  if (g_cpu_loops) {
    // Linear::forward_cpu (linear.cpp:196-215): one task per (sample, output),
    // the sum over the inputs; then the bias in a second pass
#pragma omp parallel for num_threads(g_threads) schedule(static) collapse(2)
    for (int64_t n = 0; n < B; ++n)
      for (int64_t j = 0; j < O; ++j) {
        float s = 0.f;
#pragma omp simd reduction(+ : s)
        for (int64_t i = 0; i < I; ++i) s += X[n + B * i] * W[i + I * j];
        Y[n + B * j] = s;
      }
    if (b) {
#pragma omp parallel for num_threads(g_threads) schedule(static) collapse(2)
      for (int64_t n = 0; n < B; ++n)
        for (int64_t j = 0; j < O; ++j) Y[n + B * j] += b[j];
    }
    return;
  }
  cnref_gemm_f32(0, 0, B, O, I, 1.f, X, B, W, I, 0.f, Y, B, b, 0);
}

// Sum over the batch (rows) of a ColMajor [rows, cols] matrix; the
// grad_biases_ += grad_output.sum({0}) of linear.cpp:350-352.
void cnref_column_sum(const float* in, float* out, int64_t rows, int64_t cols, int accumulate) {
  for (int64_t c = 0; c < cols; ++c) {
    const float* col = in + rows * c;
    const float s = osum(rows, [&](int64_t r) { return col[r]; });
    out[c] = accumulate ? out[c] + s : s;
  }
}

// Linear::backward_eigen (linear.cpp:335-358):
//   if trainable: grad_W += X^T dY ; grad_b += sum_batch dY
//   grad_input = dY W^T   (always, linear.cpp:357)
// accumulate=0 overwrites grad_W / grad_b instead (used for the other layers'
// zero-then-compute convention and for isolated op tests).
void cnref_linear_backward(const float* X, const float* W, const float* dY, float* gW, float* gb,
                           float* dX, int64_t B, int64_t I, int64_t O, int trainable,
                           int accumulate) {
  if (g_cpu_loops) {
    // Linear::backward_cpu (linear.cpp:289-330): one task per weight (sum
    // over the batch), per bias (the same), per input-gradient element (sum
    // over the outputs)
    if (trainable) {
#pragma omp parallel for num_threads(g_threads) schedule(static) collapse(2)
      for (int64_t i = 0; i < I; ++i)
        for (int64_t j = 0; j < O; ++j) {
          float s = 0.f;
#pragma omp simd reduction(+ : s)
          for (int64_t n = 0; n < B; ++n) s += X[n + B * i] * dY[n + B * j];
          gW[i + I * j] = accumulate ? gW[i + I * j] + s : s;
        }
      if (gb) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
        for (int64_t j = 0; j < O; ++j) {
          float s = 0.f;
#pragma omp simd reduction(+ : s)
          for (int64_t n = 0; n < B; ++n) s += dY[n + B * j];
          gb[j] = accumulate ? gb[j] + s : s;
        }
      }
    }
    if (dX) {
#pragma omp parallel for num_threads(g_threads) schedule(static) collapse(2)
      for (int64_t n = 0; n < B; ++n)
        for (int64_t i = 0; i < I; ++i) {
          float s = 0.f;
#pragma omp simd reduction(+ : s)
          for (int64_t j = 0; j < O; ++j) s += dY[n + B * j] * W[i + I * j];
          dX[n + B * i] = s;
        }
    }
    return;
  }
  if (trainable) {
    cnref_gemm_f32(1, 0, I, O, B, 1.f, X, B, dY, B, accumulate ? 1.f : 0.f, gW, I, nullptr, 0);
    if (gb) cnref_column_sum(dY, gb, B, O, accumulate);
  }
  if (dX) cnref_gemm_f32(0, 1, B, I, O, 1.f, dY, B, W, I, 0.f, dX, B, nullptr, 0);
}

void cnref_add(const float* a, const float* b, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = a[i] + b[i];
}

// Residual::forward (residual.cpp:44-87): the block's Linear layers in
// order (each caches its input), the shortcut (identity or the bias-free
// "ResProj" Linear, residual.cpp:31-36), then out + shortcut.
void cnref_residual_forward(int n_block, const int64_t* sizes, const float* const* W,
                            const float* const* b, const float* Wp, const float* x,
                            float* const* acts, float* y, int64_t B) {
  const float* h = x;
  for (int i = 0; i < n_block; ++i) {
    cnref_linear_forward(h, W[i], b[i], acts[i], B, sizes[i], sizes[i + 1]);
    h = acts[i];
  }
  const int64_t O = sizes[n_block];
  if (Wp) {
    std::vector<float> sc((size_t)(B * O));
    cnref_linear_forward(x, Wp, nullptr, sc.data(), B, sizes[0], O);
    cnref_add(h, sc.data(), y, B * O);
  } else {
    cnref_add(h, x, y, B * O);
  }
}

// Residual::backward (residual.cpp:89-131): the block's Linear backwards in
// reverse order on dY (each accumulates its grads, linear.cpp:346-352), the
// shortcut's gradient (dY itself, or the projection's backward on dY), and
// their sum.
void cnref_residual_backward(int n_block, const int64_t* sizes, const float* const* W,
                             const float* Wp, const float* x, const float* const* acts,
                             const float* dY, float* const* gW, float* const* gb, float* gWp,
                             float* dX, int64_t B) {
  std::vector<float> g(dY, dY + B * sizes[n_block]), gi;
  for (int i = n_block - 1; i >= 0; --i) {
    const float* in = i == 0 ? x : acts[i - 1];
    gi.assign((size_t)(B * sizes[i]), 0.f);
    cnref_linear_backward(in, W[i], g.data(), gW[i], gb[i], gi.data(), B, sizes[i], sizes[i + 1], 1, 1);
    g.swap(gi);
  }
  const int64_t I = sizes[0];
  if (Wp) {
    std::vector<float> gs((size_t)(B * I));
    cnref_linear_backward(x, Wp, dY, gWp, nullptr, gs.data(), B, I, sizes[n_block], 1, 1);
    cnref_add(g.data(), gs.data(), dX, B * I);
  } else {
    cnref_add(g.data(), dY, dX, B * I);
  }
}

// ReLU::forward cpu-eigen: cwiseMax(0) (relu.cpp:116-119)
void cnref_relu_forward(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = std::max(x[i], 0.0f);
}
// ReLU::backward cpu-eigen: grad * select(out > 0, 1, 0) (relu.cpp:176-182)
void cnref_relu_backward(const float* y, const float* dy, float* dx, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dx[i] = dy[i] * (y[i] > 0.0f ? 1.0f : 0.0f);
}
// Sigmoid::forward cpu-eigen (sigmoid.cpp:123-128)
void cnref_sigmoid_forward(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const float c = std::max(-500.0f, std::min(500.0f, x[i]));
    y[i] = 1.0f / (1.0f + ref_exp(-c));
  }
}
// Sigmoid::backward cpu-eigen: grad * (s * (1 - s)) (sigmoid.cpp:190-194)
void cnref_sigmoid_backward(const float* y, const float* dy, float* dx, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dx[i] = dy[i] * (y[i] * (1.0f - y[i]));
}
// Tanh::forward (tanh.cpp:100-134, cpu-eigen: .tanh())
void cnref_tanh_forward(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = ref_tanh(x[i]);
}
// Tanh::backward cpu-eigen: grad * (1 - t*t) (tanh.cpp:151-155)
void cnref_tanh_backward(const float* y, const float* dy, float* dx, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dx[i] = dy[i] * (1.0f - y[i] * y[i]);
}

// BinaryCrossEntropy::forward (binary_cross_entropy.cpp:143-184).  Targets
// are validated to {0,1} by the caller side (validate_inputs, 101-131).
float cnref_bce_forward(const float* p, const float* t, int64_t n, int reduction) {
  float total = 0.0f;
  for (int64_t i = 0; i < n; ++i) {
    const float pc = std::max(1e-7f, std::min(p[i], 1.0f - 1e-7f));
    const float tv = t[i];
    total += -(tv * ref_log(pc) + (1.0f - tv) * ref_log(1.0f - pc));
  }
  return reduction == 1 ? total : total / (float)n;
}
// BinaryCrossEntropy::backward (binary_cross_entropy.cpp:186-225): the
// denominator p*(1.0-p) is evaluated in double (the literal 1.0), the
// quotient narrowed to float, then divided by n in float for "mean".
void cnref_bce_backward(const float* p, const float* t, float* g, int64_t n, int reduction) {
  for (int64_t i = 0; i < n; ++i) {
    const float pc = std::max(1e-7f, std::min(p[i], 1.0f - 1e-7f));
    float gv = (pc - t[i]) / (pc * (1.0 - pc));
    if (reduction == 0) gv /= (float)n;
    g[i] = gv;
  }
}
// MSE::forward (mse.cpp:102-130)
float cnref_mse_forward(const float* p, const float* t, int64_t n, int reduction) {
  float s = 0.0f;
  for (int64_t i = 0; i < n; ++i) {
    const float d = p[i] - t[i];
    s += d * d;
  }
  return reduction == 0 ? s / (float)n : s;
}
// MSE::backward (mse.cpp:132-161): scale = 2/n for mean
void cnref_mse_backward(const float* p, const float* t, float* g, int64_t n, int reduction) {
  const float scale = reduction == 0 ? 2.0f / (float)n : 2.0f;
  for (int64_t i = 0; i < n; ++i) g[i] = scale * (p[i] - t[i]);
}
// SoftmaxCrossEntropy::forward (softmax_cross_entropy.cpp:118-157), ColMajor
// [B, C].  The cached softmax is exp(z - max) / sum_exp; the loss uses
// log(sum_exp + 1e-12) and is divided by the batch size for "mean".
float cnref_softmax_ce_forward(const float* z, const float* t, float* sm, int64_t B, int64_t C,
                               int reduction) {
  float total = 0.0f;
  for (int64_t b = 0; b < B; ++b) {
    float mx = z[b];
    for (int64_t c = 1; c < C; ++c) mx = std::max(mx, z[b + B * c]);
    float se = 0.0f;
    for (int64_t c = 0; c < C; ++c) {
      sm[b + B * c] = ref_exp(z[b + B * c] - mx);
      se += sm[b + B * c];
    }
    const float ls = ref_log(se + 1e-12f);
    for (int64_t c = 0; c < C; ++c) {
      sm[b + B * c] /= se;
      total -= t[b + B * c] * ((z[b + B * c] - mx) - ls);
    }
  }
  return reduction == 0 ? total / (float)B : total;
}
// SoftmaxCrossEntropy::backward (softmax_cross_entropy.cpp:159-195):
// (softmax - t) * (1/B) for mean.
void cnref_softmax_ce_backward(const float* sm, const float* t, float* g, int64_t B, int64_t C,
                               int reduction) {
  const float inv = 1.0f / (float)B;
  for (int64_t i = 0; i < B * C; ++i) {
    float v = sm[i] - t[i];
    if (reduction == 0) v *= inv;
    g[i] = v;
  }
}

// ---------------------------------------------------------------- Conv2D
// ColMajor index helpers (Eigen default layout).
static inline int64_t idx4(int64_t a, int64_t b, int64_t c, int64_t d, int64_t A, int64_t B,
                           int64_t C) {
  return a + A * (b + B * (c + C * d));
}

// Conv2D::forward (conv2d.cpp:78-136): per output element, the sum over
// (ic, kh, kw) in that order of in-bounds input * weight, then + bias.
void cnref_conv2d_forward(const float* X, const float* Wt, const float* b, float* Y, int64_t N,
                          int64_t C, int64_t H, int64_t Wd, int64_t OC, int64_t KS, int64_t S,
                          int64_t P) {
  const int64_t HO = (H + 2 * P - KS) / S + 1, WO = (Wd + 2 * P - KS) / S + 1;
  // Each output (n, oc, oh, ow) sums its (ic, kh, kw) terms in that order and
  // then adds the bias; the N samples of one (oc, oh, ow) are contiguous in
  // ColMajor [N, C, H, W], so they are evaluated side by side.
#pragma omp parallel for num_threads(g_threads) schedule(static) collapse(2)
  for (int64_t oc = 0; oc < OC; ++oc)
    for (int64_t oh = 0; oh < HO; ++oh) {
      std::vector<float> val((size_t)N);
      for (int64_t ow = 0; ow < WO; ++ow) {
        std::fill(val.begin(), val.end(), 0.0f);
        for (int64_t ic = 0; ic < C; ++ic)
          for (int64_t kh = 0; kh < KS; ++kh)
            for (int64_t kw = 0; kw < KS; ++kw) {
              const int64_t ih = oh * S - P + kh, iw = ow * S - P + kw;
              if (ih < 0 || ih >= H || iw < 0 || iw >= Wd) continue;
              const float w = Wt[idx4(oc, ic, kh, kw, OC, C, KS)];
              const float* x = X + idx4(0, ic, ih, iw, N, C, H);
              for (int64_t n = 0; n < N; ++n) val[(size_t)n] += x[n] * w;
            }
        float* y = Y + idx4(0, oc, oh, ow, N, OC, HO);
        for (int64_t n = 0; n < N; ++n) y[n] = b ? val[(size_t)n] + b[oc] : val[(size_t)n];
      }
    }
}

// Conv2D::backward (conv2d.cpp:138-198).  The reference runs one serial
// scatter loop over (n, oc, oh, ow) that accumulates gb, gW and dX.  Here the
// same sums are evaluated in passes that can run in parallel, each element
// receiving its terms in the reference's order: gW[oc, ic, kh, kw] and gb[oc]
// over (n, oh, ow); dX[n, ic, ih, iw] over (oc, oh, ow).  Grads are
// overwritten (zeroed first, 149-152).
void cnref_conv2d_backward(const float* X, const float* Wt, const float* dY, float* gW, float* gb,
                           float* dX, int64_t N, int64_t C, int64_t H, int64_t Wd, int64_t OC,
                           int64_t KS, int64_t S, int64_t P) {
  const int64_t HO = (H + 2 * P - KS) / S + 1, WO = (Wd + 2 * P - KS) / S + 1;
  // images per (channel, sample), row-major: Xi[((ic N + n) H + ih) W + iw]
  std::vector<float> Xi((size_t)(N * C * H * Wd)), Gi((size_t)(N * OC * HO * WO));
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int64_t ic = 0; ic < C; ++ic)
    for (int64_t ih = 0; ih < H; ++ih)
      for (int64_t iw = 0; iw < Wd; ++iw)
        for (int64_t n = 0; n < N; ++n)
          Xi[(size_t)(((ic * N + n) * H + ih) * Wd + iw)] = X[idx4(n, ic, ih, iw, N, C, H)];
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int64_t oc = 0; oc < OC; ++oc)
    for (int64_t oh = 0; oh < HO; ++oh)
      for (int64_t ow = 0; ow < WO; ++ow)
        for (int64_t n = 0; n < N; ++n)
          Gi[(size_t)(((oc * N + n) * HO + oh) * WO + ow)] = dY[idx4(n, oc, oh, ow, N, OC, HO)];
  if (gb) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t oc = 0; oc < OC; ++oc) {
      const float* g = Gi.data() + oc * N * HO * WO;  // (n, oh, ow) in order
      gb[oc] = osum(N * HO * WO, [&](int64_t i) { return g[i]; });
    }
  }
#pragma omp parallel for num_threads(g_threads) schedule(static) collapse(2)
  for (int64_t oc = 0; oc < OC; ++oc)
    for (int64_t ic = 0; ic < C; ++ic) {
      std::vector<float> w((size_t)(KS * KS));
      // term i = (n, oh, ow) in order adds x * g to each (kh, kw) it reaches
      osum_into(N * HO * WO, KS * KS, w.data(), [&](int64_t i, auto* acc) {
        const int64_t n = i / (HO * WO), oh = (i / WO) % HO, ow = i % WO;
        const float* xi = Xi.data() + (ic * N + n) * H * Wd;
        const float g = Gi[(size_t)((oc * N + n) * HO * WO + oh * WO + ow)];
        for (int64_t kh = 0; kh < KS; ++kh) {
          const int64_t ih = oh * S - P + kh;
          if (ih < 0 || ih >= H) continue;
          for (int64_t kw = 0; kw < KS; ++kw) {
            const int64_t iw = ow * S - P + kw;
            if (iw >= 0 && iw < Wd) acc[kh * KS + kw] += xi[ih * Wd + iw] * g;
          }
        }
      });
      for (int64_t kh = 0; kh < KS; ++kh)
        for (int64_t kw = 0; kw < KS; ++kw) gW[idx4(oc, ic, kh, kw, OC, C, KS)] = w[(size_t)(kh * KS + kw)];
    }
  // dX: the N samples of one (ic, ih, iw) are contiguous; each element takes
  // its terms in (oc, oh, ow) order (a given (oh, ow) reaches it through at
  // most one (kh, kw))
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int64_t ic = 0; ic < C; ++ic) {
    for (int64_t ih = 0; ih < H; ++ih)
      for (int64_t iw = 0; iw < Wd; ++iw) {
        float* d = dX + idx4(0, ic, ih, iw, N, C, H);
        for (int64_t n = 0; n < N; ++n) d[n] = 0.0f;
      }
    for (int64_t oc = 0; oc < OC; ++oc)
      for (int64_t oh = 0; oh < HO; ++oh)
        for (int64_t ow = 0; ow < WO; ++ow) {
          const float* g = dY + idx4(0, oc, oh, ow, N, OC, HO);
          for (int64_t kh = 0; kh < KS; ++kh)
            for (int64_t kw = 0; kw < KS; ++kw) {
              const int64_t ih = oh * S - P + kh, iw = ow * S - P + kw;
              if (ih < 0 || ih >= H || iw < 0 || iw >= Wd) continue;
              const float w = Wt[idx4(oc, ic, kh, kw, OC, C, KS)];
              float* d = dX + idx4(0, ic, ih, iw, N, C, H);
              for (int64_t n = 0; n < N; ++n) d[n] += w * g[n];
            }
        }
  }
}

// ---------------------------------------------------------------- MaxPool2D
// MaxPool2D::forward (max_pool2d.cpp:32-94)
void cnref_maxpool2d_forward(const float* X, float* Y, int32_t* idx, int64_t N, int64_t C,
                             int64_t H, int64_t W, int64_t pool, int64_t stride) {
  const int64_t HO = (H - pool) / stride + 1, WO = (W - pool) / stride + 1;
  for (int64_t n = 0; n < N; ++n)
    for (int64_t c = 0; c < C; ++c)
      for (int64_t oh = 0; oh < HO; ++oh)
        for (int64_t ow = 0; ow < WO; ++ow) {
          float mx = -std::numeric_limits<float>::infinity();
          int32_t mi = 0;
          for (int64_t ph = 0; ph < pool; ++ph)
            for (int64_t pw = 0; pw < pool; ++pw) {
              const float v = X[idx4(n, c, oh * stride + ph, ow * stride + pw, N, C, H)];
              if (v > mx) {
                mx = v;
                mi = (int32_t)(ph * pool + pw);
              }
            }
          Y[idx4(n, c, oh, ow, N, C, HO)] = mx;
          idx[idx4(n, c, oh, ow, N, C, HO)] = mi;
        }
}

// MaxPool2D::backward (max_pool2d.cpp:96-131): zeroed grad, += at argmax.
void cnref_maxpool2d_backward(const float* dY, const int32_t* idx, float* dX, int64_t N, int64_t C,
                              int64_t H, int64_t W, int64_t pool, int64_t stride) {
  const int64_t HO = (H - pool) / stride + 1, WO = (W - pool) / stride + 1;
  for (int64_t i = 0; i < N * C * H * W; ++i) dX[i] = 0.0f;
  for (int64_t n = 0; n < N; ++n)
    for (int64_t c = 0; c < C; ++c)
      for (int64_t oh = 0; oh < HO; ++oh)
        for (int64_t ow = 0; ow < WO; ++ow) {
          const int32_t k = idx[idx4(n, c, oh, ow, N, C, HO)];
          const int64_t ih = oh * stride + k / pool, iw = ow * stride + k % pool;
          dX[idx4(n, c, ih, iw, N, C, H)] += dY[idx4(n, c, oh, ow, N, C, HO)];
        }
}

// ---------------------------------------------------------------- LSTM / GRU
static inline float sigm(float x) { return 1.0f / (1.0f + ref_exp(-x)); }

// x_t = X[:, t, :] as a dense [B, I] ColMajor matrix (lstm.cpp:98-101)
static std::vector<float> slice_t(const float* X, int64_t B, int64_t S, int64_t D, int64_t t) {
  std::vector<float> x((size_t)(B * D));
  for (int64_t d = 0; d < D; ++d)
    for (int64_t n = 0; n < B; ++n) x[n + B * d] = X[n + B * t + B * S * d];
  return x;
}

// LSTM::forward (lstm.cpp:63-149): per step, gates = x_t W_ih + h W_hh, then
// i,f,o = sigmoid(. + b), g = tanh(. + b), c = f c_prev + i g, h = o tanh(c).
void cnref_lstm_forward(const float* X, const float* Wih, const float* Whh, const float* b,
                        float* Y, float* gates, float* c, float* tanh_c, int64_t B, int64_t S,
                        int64_t I, int64_t H) {
  const int64_t G = 4 * H, BS = B * S;
  std::vector<float> h((size_t)(B * H), 0.f), cp((size_t)(B * H), 0.f);
  std::vector<float> gx((size_t)(B * G)), gh((size_t)(B * G));
  for (int64_t t = 0; t < S; ++t) {
    std::vector<float> x = slice_t(X, B, S, I, t);
    cnref_gemm_f32(0, 0, B, G, I, 1.f, x.data(), B, Wih, I, 0.f, gx.data(), B, nullptr, 0);
    cnref_gemm_f32(0, 0, B, G, H, 1.f, h.data(), B, Whh, H, 0.f, gh.data(), B, nullptr, 0);
    for (int64_t n = 0; n < B; ++n)
      for (int64_t d = 0; d < H; ++d) {
        float pre[4];
        for (int q = 0; q < 4; ++q) {
          const int64_t col = d + q * H;
          pre[q] = (gx[n + B * col] + gh[n + B * col]) + b[col];
        }
        const float ig = sigm(pre[0]), fg = sigm(pre[1]), gg = ref_tanh(pre[2]), og = sigm(pre[3]);
        const float ct = fg * cp[n + B * d] + ig * gg;
        const float tc = ref_tanh(ct);
        const float ht = og * tc;
        const int64_t row = n + B * t;
        gates[row + BS * (d + 0 * H)] = ig;
        gates[row + BS * (d + 1 * H)] = fg;
        gates[row + BS * (d + 2 * H)] = gg;
        gates[row + BS * (d + 3 * H)] = og;
        c[row + BS * d] = ct;
        tanh_c[row + BS * d] = tc;
        Y[row + BS * d] = ht;
      }
    for (int64_t d = 0; d < H; ++d)
      for (int64_t n = 0; n < B; ++n) {
        h[n + B * d] = Y[n + B * t + BS * d];
        cp[n + B * d] = c[n + B * t + BS * d];
      }
  }
}

// LSTM::backward (lstm.cpp:151-253), BPTT from t = S-1 down to 0.
void cnref_lstm_backward(const float* X, const float* Wih, const float* Whh, const float* Y,
                         const float* gates, const float* c, const float* tanh_c,
                         const float* dY, float* gWih, float* gWhh, float* gb, float* dX,
                         int64_t B, int64_t S, int64_t I, int64_t H) {
  const int64_t G = 4 * H, BS = B * S;
  for (int64_t i = 0; i < I * G; ++i) gWih[i] = 0.f;
  for (int64_t i = 0; i < H * G; ++i) gWhh[i] = 0.f;
  for (int64_t i = 0; i < G; ++i) gb[i] = 0.f;
  std::vector<float> dh_next((size_t)(B * H), 0.f), dc_next((size_t)(B * H), 0.f);
  std::vector<float> dg((size_t)(B * G)), tmp_ih((size_t)(I * G)), tmp_hh((size_t)(H * G));
  std::vector<float> dx((size_t)(B * I));
  for (int64_t t = S - 1; t >= 0; --t) {
    for (int64_t n = 0; n < B; ++n)
      for (int64_t d = 0; d < H; ++d) {
        const int64_t row = n + B * t, e = n + B * d;
        const float ig = gates[row + BS * d], fg = gates[row + BS * (d + H)];
        const float gg = gates[row + BS * (d + 2 * H)], og = gates[row + BS * (d + 3 * H)];
        const float tc = tanh_c[row + BS * d];
        const float dh = dY[row + BS * d] + dh_next[e];
        const float dc = dh * og * (1.0f - tc * tc) + dc_next[e];
        const float cprev = t > 0 ? c[(n + B * (t - 1)) + BS * d] : 0.0f;
        dg[n + B * (d + 0 * H)] = dc * gg * ig * (1.0f - ig);
        dg[n + B * (d + 1 * H)] = dc * cprev * fg * (1.0f - fg);
        dg[n + B * (d + 2 * H)] = dc * ig * (1.0f - gg * gg);
        dg[n + B * (d + 3 * H)] = dh * tc * og * (1.0f - og);
        dc_next[e] = dc * fg;
      }
    if (float* tr = g_trace[CNREF_TRACE_DPRE])
      for (int64_t g = 0; g < G; ++g)
        for (int64_t n = 0; n < B; ++n) tr[(n + B * t) + BS * g] = dg[n + B * g];
    std::vector<float> x = slice_t(X, B, S, I, t);
    std::vector<float> hp = t > 0 ? slice_t(Y, B, S, H, t - 1) : std::vector<float>((size_t)(B * H), 0.f);
    cnref_gemm_f32(1, 0, I, G, B, 1.f, x.data(), B, dg.data(), B, 0.f, tmp_ih.data(), I, nullptr, 0);
    cnref_gemm_f32(1, 0, H, G, B, 1.f, hp.data(), B, dg.data(), B, 0.f, tmp_hh.data(), H, nullptr, 0);
    for (int64_t i = 0; i < I * G; ++i) gWih[i] += tmp_ih[i];
    for (int64_t i = 0; i < H * G; ++i) gWhh[i] += tmp_hh[i];
    for (int64_t g = 0; g < G; ++g)
      for (int64_t n = 0; n < B; ++n) gb[g] += dg[n + B * g];
    if (dX) {
      cnref_gemm_f32(0, 1, B, I, G, 1.f, dg.data(), B, Wih, I, 0.f, dx.data(), B, nullptr, 0);
      for (int64_t d = 0; d < I; ++d)
        for (int64_t n = 0; n < B; ++n) dX[n + B * t + BS * d] = dx[n + B * d];
    }
    cnref_gemm_f32(0, 1, B, H, G, 1.f, dg.data(), B, Whh, H, 0.f, dh_next.data(), B, nullptr, 0);
  }
}

// GRU::forward (gru.cpp:56-149).  h_gates is computed over all 3H columns, as
// the reference does, though only the z and r blocks are used.
void cnref_gru_forward(const float* X, const float* Wih, const float* Whh, const float* b,
                       float* Y, float* gates, float* rh, int64_t B, int64_t S, int64_t I,
                       int64_t H) {
  const int64_t G = 3 * H, BS = B * S;
  std::vector<float> h((size_t)(B * H), 0.f), gx((size_t)(B * G)), gh((size_t)(B * G));
  std::vector<float> rhv((size_t)(B * H)), proj((size_t)(B * H));
  for (int64_t t = 0; t < S; ++t) {
    std::vector<float> x = slice_t(X, B, S, I, t);
    cnref_gemm_f32(0, 0, B, G, I, 1.f, x.data(), B, Wih, I, 0.f, gx.data(), B, nullptr, 0);
    cnref_gemm_f32(0, 0, B, G, H, 1.f, h.data(), B, Whh, H, 0.f, gh.data(), B, nullptr, 0);
    std::vector<float> zg((size_t)(B * H)), rg((size_t)(B * H));
    for (int64_t d = 0; d < H; ++d)
      for (int64_t n = 0; n < B; ++n) {
        const int64_t e = n + B * d;
        zg[e] = sigm((gx[n + B * d] + gh[n + B * d]) + b[d]);
        rg[e] = sigm((gx[n + B * (d + H)] + gh[n + B * (d + H)]) + b[d + H]);
        rhv[e] = rg[e] * h[e];
      }
    // rh . W_hn, W_hn = columns [2H, 3H) of W_hh (gru.cpp:111-116)
    cnref_gemm_f32(0, 0, B, H, H, 1.f, rhv.data(), B, Whh + H * 2 * H, H, 0.f, proj.data(), B, nullptr, 0);
    for (int64_t d = 0; d < H; ++d)
      for (int64_t n = 0; n < B; ++n) {
        const int64_t e = n + B * d, row = n + B * t;
        const float nc = ref_tanh((gx[n + B * (d + 2 * H)] + proj[e]) + b[d + 2 * H]);
        const float ht = (1.0f - zg[e]) * nc + zg[e] * h[e];
        gates[row + BS * d] = zg[e];
        gates[row + BS * (d + H)] = rg[e];
        gates[row + BS * (d + 2 * H)] = nc;
        rh[row + BS * d] = rhv[e];
        Y[row + BS * d] = ht;
      }
    for (int64_t d = 0; d < H; ++d)
      for (int64_t n = 0; n < B; ++n) h[n + B * d] = Y[n + B * t + BS * d];
  }
}

// GRU::backward (gru.cpp:151-297)
void cnref_gru_backward(const float* X, const float* Wih, const float* Whh, const float* Y,
                        const float* gates, const float* rh, const float* dY, float* gWih,
                        float* gWhh, float* gb, float* dX, int64_t B, int64_t S, int64_t I,
                        int64_t H) {
  const int64_t G = 3 * H, BS = B * S;
  for (int64_t i = 0; i < I * G; ++i) gWih[i] = 0.f;
  for (int64_t i = 0; i < H * G; ++i) gWhh[i] = 0.f;
  for (int64_t i = 0; i < G; ++i) gb[i] = 0.f;
  std::vector<float> dh_next((size_t)(B * H), 0.f), dg((size_t)(B * G)), dhp((size_t)(B * H));
  std::vector<float> dn_raw((size_t)(B * H)), d_rh((size_t)(B * H)), dzr((size_t)(B * H));
  std::vector<float> tmp_ih((size_t)(I * G)), tmp((size_t)(H * G)), dx((size_t)(B * I));
  const float* Whn = Whh + H * 2 * H;
  for (int64_t t = S - 1; t >= 0; --t) {
    std::vector<float> hp = t > 0 ? slice_t(Y, B, S, H, t - 1) : std::vector<float>((size_t)(B * H), 0.f);
    for (int64_t d = 0; d < H; ++d)
      for (int64_t n = 0; n < B; ++n) {
        const int64_t e = n + B * d, row = n + B * t;
        const float zg = gates[row + BS * d], nc = gates[row + BS * (d + 2 * H)];
        const float dh = dY[row + BS * d] + dh_next[e];
        const float dn = dh * (1.0f - zg);
        const float dz = dh * (hp[e] - nc);
        dhp[e] = dh * zg;
        dn_raw[e] = dn * (1.0f - nc * nc);
        dg[n + B * d] = dz * zg * (1.0f - zg);
        dg[n + B * (d + 2 * H)] = dn_raw[e];
      }
    // d_rh = dn_raw W_hn^T
    cnref_gemm_f32(0, 1, B, H, H, 1.f, dn_raw.data(), B, Whn, H, 0.f, d_rh.data(), B, nullptr, 0);
    for (int64_t d = 0; d < H; ++d)
      for (int64_t n = 0; n < B; ++n) {
        const int64_t e = n + B * d, row = n + B * t;
        const float rg = gates[row + BS * (d + H)];
        const float dr = d_rh[e] * hp[e];
        dg[n + B * (d + H)] = dr * rg * (1.0f - rg);
        dhp[e] += d_rh[e] * rg;
      }
    if (float* tr = g_trace[CNREF_TRACE_DPRE])
      for (int64_t g = 0; g < G; ++g)
        for (int64_t n = 0; n < B; ++n) tr[(n + B * t) + BS * g] = dg[n + B * g];
    std::vector<float> x = slice_t(X, B, S, I, t);
    cnref_gemm_f32(1, 0, I, G, B, 1.f, x.data(), B, dg.data(), B, 0.f, tmp_ih.data(), I, nullptr, 0);
    for (int64_t i = 0; i < I * G; ++i) gWih[i] += tmp_ih[i];
    // z and r blocks against h_prev, n block against r*h_prev (gru.cpp:240-251)
    std::vector<float> rht = slice_t(rh, B, S, H, t);
    cnref_gemm_f32(1, 0, H, 2 * H, B, 1.f, hp.data(), B, dg.data(), B, 0.f, tmp.data(), H, nullptr, 0);
    for (int64_t i = 0; i < H * 2 * H; ++i) gWhh[i] += tmp[i];
    cnref_gemm_f32(1, 0, H, H, B, 1.f, rht.data(), B, dg.data() + B * 2 * H, B, 0.f, tmp.data(), H,
                   nullptr, 0);
    for (int64_t i = 0; i < H * H; ++i) gWhh[H * 2 * H + i] += tmp[i];
    for (int64_t g = 0; g < G; ++g)
      for (int64_t n = 0; n < B; ++n) gb[g] += dg[n + B * g];
    if (dX) {
      cnref_gemm_f32(0, 1, B, I, G, 1.f, dg.data(), B, Wih, I, 0.f, dx.data(), B, nullptr, 0);
      for (int64_t d = 0; d < I; ++d)
        for (int64_t n = 0; n < B; ++n) dX[n + B * t + BS * d] = dx[n + B * d];
    }
    // dh_next = dh_prev + dgates[z,r] W_hh[:, 0:2H]^T (gru.cpp:262-277)
    cnref_gemm_f32(0, 1, B, H, 2 * H, 1.f, dg.data(), B, Whh, H, 0.f, dzr.data(), B, nullptr, 0);
    for (int64_t e = 0; e < B * H; ++e) dh_next[e] = dhp[e] + dzr[e];
  }
}

// ---------------------------------------------------------------- Embedding
// Embedding::forward cpu-eigen (embedding.cpp:79-95)
int cnref_embedding_forward(const int32_t* ids, const float* W, float* out, int64_t B, int64_t S,
                            int64_t V, int64_t D) {
  for (int64_t n = 0; n < B; ++n)
    for (int64_t s = 0; s < S; ++s) {
      const int32_t id = ids[n + B * s];
      if (id < 0 || id >= V) return -1;
      for (int64_t d = 0; d < D; ++d) out[n + B * s + B * S * d] = W[id + V * d];
    }
  return 0;
}
// Embedding::backward cpu-eigen (embedding.cpp:108, 163-175)
void cnref_embedding_backward(const int32_t* ids, const float* dY, float* gW, int64_t B, int64_t S,
                              int64_t V, int64_t D) {
  for (int64_t i = 0; i < V * D; ++i) gW[i] = 0.0f;
  for (int64_t n = 0; n < B; ++n)
    for (int64_t s = 0; s < S; ++s) {
      const int32_t id = ids[n + B * s];
      for (int64_t d = 0; d < D; ++d) gW[id + V * d] += dY[n + B * s + B * S * d];
    }
}

// ---------------------------------------------------------------- MHA
// sample n of a [B,S,D] tensor as a dense [S,D] ColMajor matrix
static std::vector<float> sample_sd(const float* x, int64_t B, int64_t S, int64_t D, int64_t n) {
  std::vector<float> m((size_t)(S * D));
  for (int64_t d = 0; d < D; ++d)
    for (int64_t s = 0; s < S; ++s) m[s + S * d] = x[n + B * s + B * S * d];
  return m;
}

// MultiHeadAttention::forward cpu-eigen branch (attention.cpp:165-218)
void cnref_mha_forward(const float* q, const float* k, const float* v, const float* Wq,
                       const float* Wk, const float* Wv, const float* Wo, float* out, float* attn,
                       int64_t B, int64_t S, int64_t D, int64_t heads) {
  const float scale = 1.0f / std::sqrt(static_cast<float>(D / heads));
  std::vector<float> Qp((size_t)(S * D)), Kp((size_t)(S * D)), Vp((size_t)(S * D));
  std::vector<float> sc((size_t)(S * S)), A((size_t)(S * S)), ctx((size_t)(S * D)), o((size_t)(S * D));
  for (int64_t n = 0; n < B; ++n) {
    auto Q = sample_sd(q, B, S, D, n), K = sample_sd(k, B, S, D, n), V = sample_sd(v, B, S, D, n);
    cnref_gemm_f32(0, 0, S, D, D, 1.f, Q.data(), S, Wq, D, 0.f, Qp.data(), S, nullptr, 0);
    cnref_gemm_f32(0, 0, S, D, D, 1.f, K.data(), S, Wk, D, 0.f, Kp.data(), S, nullptr, 0);
    cnref_gemm_f32(0, 0, S, D, D, 1.f, V.data(), S, Wv, D, 0.f, Vp.data(), S, nullptr, 0);
    // scores = Qp Kp^T, then * scale (189)
    cnref_gemm_f32(0, 1, S, S, D, 1.f, Qp.data(), S, Kp.data(), S, 0.f, sc.data(), S, nullptr, 0);
    for (auto& x : sc) x = x * scale;
    for (int64_t i = 0; i < S; ++i) {  // row softmax (191-205)
      float mx = sc[i];
      for (int64_t j = 1; j < S; ++j) mx = std::max(mx, sc[i + S * j]);
      float sum = 0.0f;
      for (int64_t j = 0; j < S; ++j) {
        A[i + S * j] = ref_exp(sc[i + S * j] - mx);
        sum += A[i + S * j];
      }
      for (int64_t j = 0; j < S; ++j) A[i + S * j] /= sum;
    }
    for (int64_t j = 0; j < S; ++j)
      for (int64_t i = 0; i < S; ++i) attn[n + B * i + B * S * j] = A[i + S * j];
    cnref_gemm_f32(0, 0, S, D, S, 1.f, A.data(), S, Vp.data(), S, 0.f, ctx.data(), S, nullptr, 0);
    cnref_gemm_f32(0, 0, S, D, D, 1.f, ctx.data(), S, Wo, D, 0.f, o.data(), S, nullptr, 0);
    for (int64_t d = 0; d < D; ++d)
      for (int64_t s = 0; s < S; ++s) out[n + B * s + B * S * d] = o[s + S * d];
  }
}

// MultiHeadAttention::backward cpu-eigen branch (attention.cpp:503-569)
void cnref_mha_backward(const float* q, const float* k, const float* v, const float* Wq,
                        const float* Wk, const float* Wv, const float* Wo, const float* attn,
                        const float* dY, float* gWq, float* gWk, float* gWv, float* gWo,
                        float* dX, int64_t B, int64_t S, int64_t D, int64_t heads) {
  const float scale = 1.0f / std::sqrt(static_cast<float>(D / heads));
  for (int64_t i = 0; i < D * D; ++i) gWq[i] = gWk[i] = gWv[i] = gWo[i] = 0.0f;
  const size_t SD = (size_t)(S * D), SS = (size_t)(S * S), DD = (size_t)(D * D);
  std::vector<float> Qp(SD), Kp(SD), Vp(SD), ctx(SD), gctx(SD), gA(SS), gVp(SD), gS(SS), gQp(SD),
      gKp(SD), gQ(SD), gK(SD), gV(SD), A(SS), tmp(DD);
  for (int64_t n = 0; n < B; ++n) {
    auto G = sample_sd(dY, B, S, D, n);
    auto Q = sample_sd(q, B, S, D, n), K = sample_sd(k, B, S, D, n), V = sample_sd(v, B, S, D, n);
    for (int64_t j = 0; j < S; ++j)
      for (int64_t i = 0; i < S; ++i) A[i + S * j] = attn[n + B * i + B * S * j];
    cnref_gemm_f32(0, 0, S, D, D, 1.f, Q.data(), S, Wq, D, 0.f, Qp.data(), S, nullptr, 0);
    cnref_gemm_f32(0, 0, S, D, D, 1.f, K.data(), S, Wk, D, 0.f, Kp.data(), S, nullptr, 0);
    cnref_gemm_f32(0, 0, S, D, D, 1.f, V.data(), S, Wv, D, 0.f, Vp.data(), S, nullptr, 0);
    cnref_gemm_f32(0, 0, S, D, S, 1.f, A.data(), S, Vp.data(), S, 0.f, ctx.data(), S, nullptr, 0);
    cnref_gemm_f32(0, 1, S, D, D, 1.f, G.data(), S, Wo, D, 0.f, gctx.data(), S, nullptr, 0);
    cnref_gemm_f32(1, 0, D, D, S, 1.f, ctx.data(), S, G.data(), S, 0.f, tmp.data(), D, nullptr, 0);
    for (size_t i = 0; i < DD; ++i) gWo[i] += tmp[i];
    cnref_gemm_f32(0, 1, S, S, D, 1.f, gctx.data(), S, Vp.data(), S, 0.f, gA.data(), S, nullptr, 0);
    cnref_gemm_f32(1, 0, S, D, S, 1.f, A.data(), S, gctx.data(), S, 0.f, gVp.data(), S, nullptr, 0);
    for (int64_t i = 0; i < S; ++i) {  // softmax Jacobian rows (541-549)
      float dot = 0.0f;
      for (int64_t j = 0; j < S; ++j) dot += gA[i + S * j] * A[i + S * j];
      for (int64_t j = 0; j < S; ++j) gS[i + S * j] = A[i + S * j] * (gA[i + S * j] - dot);
    }
    for (auto& x : gS) x = x * scale;
    cnref_gemm_f32(0, 0, S, D, S, 1.f, gS.data(), S, Kp.data(), S, 0.f, gQp.data(), S, nullptr, 0);
    cnref_gemm_f32(1, 0, S, D, S, 1.f, gS.data(), S, Qp.data(), S, 0.f, gKp.data(), S, nullptr, 0);
    cnref_gemm_f32(0, 1, S, D, D, 1.f, gQp.data(), S, Wq, D, 0.f, gQ.data(), S, nullptr, 0);
    cnref_gemm_f32(1, 0, D, D, S, 1.f, Q.data(), S, gQp.data(), S, 0.f, tmp.data(), D, nullptr, 0);
    for (size_t i = 0; i < DD; ++i) gWq[i] += tmp[i];
    cnref_gemm_f32(0, 1, S, D, D, 1.f, gKp.data(), S, Wk, D, 0.f, gK.data(), S, nullptr, 0);
    cnref_gemm_f32(1, 0, D, D, S, 1.f, K.data(), S, gKp.data(), S, 0.f, tmp.data(), D, nullptr, 0);
    for (size_t i = 0; i < DD; ++i) gWk[i] += tmp[i];
    cnref_gemm_f32(0, 1, S, D, D, 1.f, gVp.data(), S, Wv, D, 0.f, gV.data(), S, nullptr, 0);
    cnref_gemm_f32(1, 0, D, D, S, 1.f, V.data(), S, gVp.data(), S, 0.f, tmp.data(), D, nullptr, 0);
    for (size_t i = 0; i < DD; ++i) gWv[i] += tmp[i];
    for (int64_t d = 0; d < D; ++d)
      for (int64_t s2 = 0; s2 < S; ++s2)
        dX[n + B * s2 + B * S * d] = gQ[s2 + S * d] + gK[s2 + S * d] + gV[s2 + S * d];
    const std::vector<float>* sample_tr[4] = {&gQp, &gKp, &gVp, &ctx};
    for (int slot = CNREF_TRACE_GQP; slot <= CNREF_TRACE_CTX; ++slot)
      if (float* tr = g_trace[slot]) {
        const std::vector<float>& src = *sample_tr[slot - CNREF_TRACE_GQP];
        for (int64_t d = 0; d < D; ++d)
          for (int64_t s2 = 0; s2 < S; ++s2) tr[n + B * s2 + B * S * d] = src[(size_t)(s2 + S * d)];
      }
  }
}

// ---------------------------------------------------------------- BatchNorm
// BatchNorm::forward cpu-eigen, training (batch_norm.cpp:282-318)
void cnref_batchnorm_forward(const float* x, float* y, float* xhat, const float* gamma,
                             const float* beta, float* running_mean, float* running_var,
                             float* batch_mean, float* batch_var, int64_t N, int64_t F,
                             float momentum, float eps) {
  const float inv_batch = 1.0f / static_cast<float>(N);
  for (int64_t f = 0; f < F; ++f) {
    const float* xc = x + N * f;
    float m = osum(N, [&](int64_t n) { return xc[n]; });
    m *= inv_batch;
    float var = osum(N, [&](int64_t n) {
      const float diff = xc[n] - m;
      return diff * diff;
    });
    var *= inv_batch;
    batch_mean[f] = m;
    batch_var[f] = var;
    for (int64_t n = 0; n < N; ++n) {
      xhat[n + N * f] = (x[n + N * f] - m) / std::sqrt(var + eps);
      y[n + N * f] = gamma[f] * xhat[n + N * f] + beta[f];
    }
    running_mean[f] = (1.0f - momentum) * running_mean[f] + momentum * m;
    running_var[f] = (1.0f - momentum) * running_var[f] + momentum * var;
  }
}
// BatchNorm::backward (batch_norm.cpp:333-388)
void cnref_batchnorm_backward(const float* dY, const float* x, const float* xhat,
                              const float* gamma, const float* batch_mean, const float* batch_var,
                              float* ggamma, float* gbeta, float* dX, int64_t N, int64_t F,
                              float eps) {
  const float inv_batch = 1.0f / static_cast<float>(N);
  for (int64_t f = 0; f < F; ++f) {
    const float* dy = dY + N * f;
    ggamma[f] = osum(N, [&](int64_t n) { return dy[n] * xhat[n + N * f]; });
    gbeta[f] = osum(N, [&](int64_t n) { return dy[n]; });
    const float inv_std = 1.0f / std::sqrt(batch_var[f] + eps);
    const float dvar = osum(N, [&](int64_t n) {
      const float dxh = dy[n] * gamma[f];
      const float xmu = x[n + N * f] - batch_mean[f];
      return dxh * xmu * (-0.5f) * inv_std * inv_std * inv_std;
    });
    const float dmean = osum(N, [&](int64_t n) { return dy[n] * gamma[f] * (-inv_std); });
    for (int64_t n = 0; n < N; ++n) {
      const float dxh = dY[n + N * f] * gamma[f];
      const float xmu = x[n + N * f] - batch_mean[f];
      dX[n + N * f] = dxh * inv_std + dvar * 2.0f * xmu * inv_batch + dmean * inv_batch;
    }
  }
}

// ---------------------------------------------------------------- GELU
void cnref_gelu_forward(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const double v = x[i];
    y[i] = (float)(0.5 * v * (1.0 + std::erf(v * 0.70710678118654752440)));
  }
}
void cnref_gelu_backward(const float* x, const float* dy, float* dx, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const double v = x[i];
    const double cdf = 0.5 * (1.0 + std::erf(v * 0.70710678118654752440));
    const double pdf = 0.39894228040143267794 * std::exp(-0.5 * v * v);
    dx[i] = (float)((double)dy[i] * (cdf + v * pdf));
  }
}

// ---------------------------------------------------------------- MeanPool1D
// mean over the sequence (mean_pool1d.cpp:37-42: Eigen mean = sum / S)
void cnref_meanpool1d_forward(const float* x, float* y, int64_t B, int64_t S, int64_t D) {
  for (int64_t d = 0; d < D; ++d)
    for (int64_t b = 0; b < B; ++b) {
      const float sum = osum(S, [&](int64_t s) { return x[b + B * s + B * S * d]; });
      y[b + B * d] = sum / static_cast<float>(S);
    }
}
// mean_pool1d.cpp:97-104: grad_input = grad_output * (1/S)
void cnref_meanpool1d_backward(const float* dy, float* dx, int64_t B, int64_t S, int64_t D) {
  const float inv_S = 1.0f / static_cast<float>(S);
  for (int64_t d = 0; d < D; ++d)
    for (int64_t s = 0; s < S; ++s)
      for (int64_t b = 0; b < B; ++b) dx[b + B * s + B * S * d] = dy[b + B * d] * inv_S;
}

// Adam::update (adam.cpp:98-133), per element in order.
void cnref_adam_step(float* W, const float* g, float* m, float* v, int64_t n, float lr, float b1,
                     float b2, float eps, float bc1, float bc2) {
  for (int64_t i = 0; i < n; ++i) {
    m[i] = b1 * m[i] + (1.0f - b1) * g[i];
    v[i] = b2 * v[i] + (1.0f - b2) * g[i] * g[i];
    const float mh = m[i] / bc1;
    const float vh = v[i] / bc2;
    W[i] -= lr * mh / (std::sqrt(vh) + eps);
  }
}

// adam.cpp:121-122: 1.0f - std::pow(beta, static_cast<float>(t))
float cnref_bias_correction(float beta, int t) {
  return 1.0f - std::pow(beta, static_cast<float>(t));
}

}  // extern "C"
