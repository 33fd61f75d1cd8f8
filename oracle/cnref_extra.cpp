// cnref_extra.cpp — CPU oracle, part 2: the reference's device ops off the
// BASELINE configs (LeakyReLU, Softmax, CategoricalCrossEntropy, MAE, Huber,
// SGD / Momentum / Adagrad / RMSProp, Dropout, GlobalAvg/MaxPool2D, Elman RNN).
//
// TEST INFRASTRUCTURE ONLY, like cnref.cpp: plain C++17 loops restating the
// reference's cpu / cpu-eigen branches, each citing the file:line it follows.
// Layout is Eigen ColMajor (first index fastest).  Built without FMA
// contraction, so every fp32 operation rounds once.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <limits>
#include <vector>

#include "cnref.h"
#include "cnref_fn.hpp"

extern "C" {

// ---------------------------------------------------------------- LeakyReLU
// leacky_relu.cpp:93-156 (2-D; 4-D at 158-229): y = x > 0 ? x : alpha * x; dx = x > 0 ? dy : alpha * dy
// (the backward reads the cached INPUT).
void cnref_leaky_relu_forward(const float* x, float* y, int64_t n, float alpha) {
  for (int64_t i = 0; i < n; ++i) y[i] = x[i] > 0.0f ? x[i] : alpha * x[i];
}
void cnref_leaky_relu_backward(const float* x, const float* dy, float* dx, int64_t n, float alpha) {
  for (int64_t i = 0; i < n; ++i) dx[i] = x[i] > 0.0f ? dy[i] : alpha * dy[i];
}

// ---------------------------------------------------------------- Softmax
// softmax.cpp:105-162 (2-D) and 209-270 (4-D): softmax over the LAST dimension.
// A ColMajor tensor whose last dimension has L entries is R = size / L rows
// with element (r, j) at r + R*j.  Per row: max from j = 0, exp(x - max),
// sum in j order, then divide.
void cnref_softmax_forward(const float* x, float* y, int64_t R, int64_t L) {
  for (int64_t r = 0; r < R; ++r) {
    float mx = x[r];
    for (int64_t j = 1; j < L; ++j) mx = std::max(mx, x[r + R * j]);
    float s = 0.0f;
    for (int64_t j = 0; j < L; ++j) {
      y[r + R * j] = ref_exp(x[r + R * j] - mx);
      s += y[r + R * j];
    }
    for (int64_t j = 0; j < L; ++j) y[r + R * j] /= s;
  }
}
// softmax.cpp:164-207 (2-D), 272-323 (4-D): dot = sum_j dy*y (j order); dx = y * (dy - dot)
void cnref_softmax_backward(const float* y, const float* dy, float* dx, int64_t R, int64_t L) {
  for (int64_t r = 0; r < R; ++r) {
    float dot = 0.0f;
    for (int64_t j = 0; j < L; ++j) dot += dy[r + R * j] * y[r + R * j];
    for (int64_t j = 0; j < L; ++j) dx[r + R * j] = y[r + R * j] * (dy[r + R * j] - dot);
  }
}

// ---------------------------------------------------------------- CCE
// categorical_cross_entropy.cpp:167-259 (float-target forward; the int-label
// and 3-D overloads at 141-165, 261-293 build one-hot targets and call it).  targets_used
// receives t * (1 - ls) + ls / C when ls > 0 (else a copy of t); sm receives
// the softmax of the logits (from_logits) or a copy of the predictions.
// loss = sum_b sum_j -t * log(clip(p, 1e-15, 1 - 1e-15)), / B for "mean".
float cnref_cce_forward(const float* pred, const float* t, float* sm, float* targets_used, int64_t B,
                        int64_t C, int from_logits, float label_smoothing, int reduction) {
  const int64_t n = B * C;
  if (label_smoothing > 0.0f) {
    const float sf = label_smoothing / (float)C;
    for (int64_t i = 0; i < n; ++i) targets_used[i] = t[i] * (1.0f - label_smoothing) + sf;
  } else {
    for (int64_t i = 0; i < n; ++i) targets_used[i] = t[i];
  }
  if (from_logits) {
    for (int64_t b = 0; b < B; ++b) {
      float mx = pred[b];
      for (int64_t j = 1; j < C; ++j)
        if (pred[b + B * j] > mx) mx = pred[b + B * j];
      float se = 0.0f;
      for (int64_t j = 0; j < C; ++j) {
        const float e = ref_exp(pred[b + B * j] - mx);
        sm[b + B * j] = e;
        se += e;
      }
      for (int64_t j = 0; j < C; ++j) sm[b + B * j] /= se;
    }
  } else {
    for (int64_t i = 0; i < n; ++i) sm[i] = pred[i];
  }
  const float eps = 1e-15f;
  float total = 0.0f;
  for (int64_t b = 0; b < B; ++b) {
    float sample = 0.0f;
    for (int64_t j = 0; j < C; ++j) {
      const float p = std::max(eps, std::min(1.0f - eps, sm[b + B * j]));
      sample -= targets_used[b + B * j] * ref_log(p);
    }
    total += sample;
  }
  return reduction == 0 ? total / (float)B : total;
}
// categorical_cross_entropy.cpp:316-380 backward: from_logits g = sm - t; else
// g = -t / clip(p); "mean" then divides every entry by B.
void cnref_cce_backward(const float* sm, const float* targets_used, float* g, int64_t B, int64_t C,
                        int from_logits, int reduction) {
  const int64_t n = B * C;
  const float eps = 1e-15f;
  for (int64_t i = 0; i < n; ++i) {
    if (from_logits) {
      g[i] = sm[i] - targets_used[i];
    } else {
      const float p = std::max(eps, std::min(1.0f - eps, sm[i]));
      g[i] = -targets_used[i] / p;
    }
    if (reduction == 0) g[i] /= (float)B;
  }
}

// ---------------------------------------------------------------- MAE, Huber
// mae.cpp:102-160 MAE::forward/backward: mean |p - t| over all n; grad = sign(d) * scale,
// scale = 1 / n (0 where d == 0).
float cnref_mae_forward(const float* p, const float* t, int64_t n, int reduction) {
  float s = 0.0f;
  for (int64_t i = 0; i < n; ++i) s += std::fabs(p[i] - t[i]);
  return reduction == 0 ? s / (float)n : s;
}
void cnref_mae_backward(const float* p, const float* t, float* g, int64_t n, int reduction) {
  const float scale = reduction == 0 ? 1.0f / (float)n : 1.0f;
  for (int64_t i = 0; i < n; ++i) {
    const float d = p[i] - t[i];
    g[i] = d > 0.0f ? scale : (d < 0.0f ? -scale : 0.0f);
  }
}
// huber.cpp:104-178 Huber::forward/backward: |d| <= delta: 0.5 d^2 (grad scale * d),
// else delta (|d| - 0.5 delta) (grad scale * delta * sign(d), sign(0) = -1
// is unreachable there).
float cnref_huber_forward(const float* p, const float* t, int64_t n, float delta, int reduction) {
  float s = 0.0f;
  for (int64_t i = 0; i < n; ++i) {
    const float d = p[i] - t[i];
    const float a = std::fabs(d);
    if (a <= delta)
      s += 0.5f * d * d;
    else
      s += delta * (a - 0.5f * delta);
  }
  return reduction == 0 ? s / (float)n : s;
}
void cnref_huber_backward(const float* p, const float* t, float* g, int64_t n, float delta, int reduction) {
  const float scale = reduction == 0 ? 1.0f / (float)n : 1.0f;
  for (int64_t i = 0; i < n; ++i) {
    const float d = p[i] - t[i];
    if (std::fabs(d) <= delta)
      g[i] = scale * d;
    else
      g[i] = scale * delta * (d > 0.0f ? 1.0f : -1.0f);
  }
}

// ---------------------------------------------------------------- optimizers
// sgd.cpp:54-68: W -= lr * g
void cnref_sgd_step(float* W, const float* g, int64_t n, float lr) {
  for (int64_t i = 0; i < n; ++i) W[i] -= lr * g[i];
}
// momentum.cpp:81-104: vel = mu * vel - lr * g; W += vel
void cnref_momentum_step(float* W, const float* g, float* vel, int64_t n, float lr, float mu) {
  for (int64_t i = 0; i < n; ++i) {
    vel[i] = mu * vel[i] - lr * g[i];
    W[i] += vel[i];
  }
}
// adagrad.cpp:83-106: acc += g * g; W -= lr * g / (sqrt(acc) + eps)
void cnref_adagrad_step(float* W, const float* g, float* acc, int64_t n, float lr, float eps) {
  for (int64_t i = 0; i < n; ++i) {
    acc[i] += g[i] * g[i];
    W[i] -= lr * g[i] / (std::sqrt(acc[i]) + eps);
  }
}
// mrs_prop.cpp:83-106: s = rho * s + (1 - rho) * g * g; W -= lr * g / (sqrt(s) + eps)
void cnref_rmsprop_step(float* W, const float* g, float* s, int64_t n, float lr, float rho, float eps) {
  for (int64_t i = 0; i < n; ++i) {
    s[i] = rho * s[i] + (1.0f - rho) * g[i] * g[i];
    W[i] -= lr * g[i] / (std::sqrt(s[i]) + eps);
  }
}

// ---------------------------------------------------------------- Dropout
// dropout.cpp:140-196 (2-D), 197-270 (4-D): out = x * mask * scale (forward and backward alike);
// mask entries are 0 or 1, scale = 1 / (1 - p).  The reference draws the mask
// from an unseeded std::mt19937 (dropout.cpp:19-21), so parity is on the
// arithmetic given a mask.
void cnref_dropout_apply(const float* x, const float* mask, float* y, int64_t n, float scale) {
  for (int64_t i = 0; i < n; ++i) y[i] = x[i] * mask[i] * scale;
}

// ---------------------------------------------------------------- global pools
// global_pool.cpp:111-159 GlobalAvgPool2D::forward: per (n, c), sum over h (outer),
// w (inner) in order, times inv_spatial = 1 / (H * W); X [N, C, H, W] ColMajor.
void cnref_global_avgpool_forward(const float* X, float* Y, int64_t N, int64_t C, int64_t H, int64_t W) {
  const float inv = 1.0f / (float)(H * W);
  for (int64_t n = 0; n < N; ++n)
    for (int64_t c = 0; c < C; ++c) {
      float s = 0.0f;
      for (int64_t h = 0; h < H; ++h)
        for (int64_t w = 0; w < W; ++w) s += X[n + N * (c + C * (h + H * w))];
      Y[n + N * c] = s * inv;
    }
}
// global_pool.cpp:161-210 GlobalAvgPool2D::backward: every input of (n, c) gets dY(n, c) * inv_spatial
void cnref_global_avgpool_backward(const float* dY, float* dX, int64_t N, int64_t C, int64_t H, int64_t W) {
  const float inv = 1.0f / (float)(H * W);
  for (int64_t n = 0; n < N; ++n)
    for (int64_t c = 0; c < C; ++c) {
      const float g = dY[n + N * c] * inv;
      for (int64_t h = 0; h < H; ++h)
        for (int64_t w = 0; w < W; ++w) dX[n + N * (c + C * (h + H * w))] = g;
    }
}
// global_pool.cpp:305-373 GlobalMaxPool2D::forward: scan h (outer), w (inner) from -inf with strict >,
// first maximum wins; argmax kept as (h, w) int32 [N, C] tensors.
void cnref_global_maxpool_forward(const float* X, float* Y, int32_t* ah, int32_t* aw, int64_t N,
                                  int64_t C, int64_t H, int64_t W) {
  for (int64_t n = 0; n < N; ++n)
    for (int64_t c = 0; c < C; ++c) {
      float mx = -std::numeric_limits<float>::infinity();
      int32_t bh = 0, bw = 0;
      for (int64_t h = 0; h < H; ++h)
        for (int64_t w = 0; w < W; ++w) {
          const float v = X[n + N * (c + C * (h + H * w))];
          if (v > mx) {
            mx = v;
            bh = (int32_t)h;
            bw = (int32_t)w;
          }
        }
      Y[n + N * c] = mx;
      ah[n + N * c] = bh;
      aw[n + N * c] = bw;
    }
}
// global_pool.cpp:375-395 GlobalMaxPool2D::backward: zeros, then dX(n, c, ah, aw) = dY(n, c)
void cnref_global_maxpool_backward(const float* dY, const int32_t* ah, const int32_t* aw, float* dX,
                                   int64_t N, int64_t C, int64_t H, int64_t W) {
  std::fill(dX, dX + N * C * H * W, 0.0f);
  for (int64_t n = 0; n < N; ++n)
    for (int64_t c = 0; c < C; ++c)
      dX[n + N * (c + C * (ah[n + N * c] + H * aw[n + N * c]))] = dY[n + N * c];
}

// ---------------------------------------------------------------- Elman RNN
// rnn.cpp:48-100 forward: h_0 = 0; per t: pre = x_t W_ih + h_{t-1} W_hh (two
// contractions, then added), h_t = tanh(pre + b).  X [B, S, I], Y [B, S, H].
static std::vector<float> rnn_slice(const float* T, int64_t B, int64_t S, int64_t D, int64_t t) {
  std::vector<float> out((size_t)(B * D));
  for (int64_t d = 0; d < D; ++d)
    for (int64_t n = 0; n < B; ++n) out[(size_t)(n + B * d)] = T[n + B * t + B * S * d];
  return out;
}
void cnref_rnn_forward(const float* X, const float* Wih, const float* Whh, const float* b, float* Y,
                       int64_t B, int64_t S, int64_t I, int64_t H) {
  std::vector<float> h((size_t)(B * H), 0.0f), xw((size_t)(B * H)), hw((size_t)(B * H));
  for (int64_t t = 0; t < S; ++t) {
    std::vector<float> x = rnn_slice(X, B, S, I, t);
    cnref_gemm_f32(0, 0, B, H, I, 1.f, x.data(), B, Wih, I, 0.f, xw.data(), B, nullptr, 0);
    cnref_gemm_f32(0, 0, B, H, H, 1.f, h.data(), B, Whh, H, 0.f, hw.data(), B, nullptr, 0);
    for (int64_t d = 0; d < H; ++d)
      for (int64_t n = 0; n < B; ++n) {
        const float v = ref_tanh((xw[(size_t)(n + B * d)] + hw[(size_t)(n + B * d)]) + b[d]);
        h[(size_t)(n + B * d)] = v;
        Y[n + B * t + B * S * d] = v;
      }
  }
}
// rnn.cpp:102-171 backward (grads overwrite): per t from S-1 down:
// dh = dY_t + dh_next; dtanh = dh * (1 - h_t^2); gW_ih += x_t^T dtanh;
// gW_hh += h_{t-1}^T dtanh; gb += colsum(dtanh); dX_t = dtanh W_ih^T;
// dh_next = dtanh W_hh^T.
void cnref_rnn_backward(const float* X, const float* Wih, const float* Whh, const float* Y,
                        const float* dY, float* gWih, float* gWhh, float* gb, float* dX, int64_t B,
                        int64_t S, int64_t I, int64_t H) {
  std::fill(gWih, gWih + I * H, 0.0f);
  std::fill(gWhh, gWhh + H * H, 0.0f);
  std::fill(gb, gb + H, 0.0f);
  std::vector<float> dh_next((size_t)(B * H), 0.0f), dt((size_t)(B * H)), dx((size_t)(B * I));
  for (int64_t t = S - 1; t >= 0; --t) {
    std::vector<float> ht = rnn_slice(Y, B, S, H, t);
    std::vector<float> hp = t > 0 ? rnn_slice(Y, B, S, H, t - 1) : std::vector<float>((size_t)(B * H), 0.0f);
    std::vector<float> x = rnn_slice(X, B, S, I, t);
    for (int64_t d = 0; d < H; ++d)
      for (int64_t n = 0; n < B; ++n) {
        const size_t k = (size_t)(n + B * d);
        const float dh = dY[n + B * t + B * S * d] + dh_next[k];
        dt[k] = dh * (1.0f - ht[k] * ht[k]);
      }
    if (float* tr = cnref_trace(CNREF_TRACE_DPRE))
      for (int64_t d = 0; d < H; ++d)
        for (int64_t n = 0; n < B; ++n) tr[(n + B * t) + B * S * d] = dt[(size_t)(n + B * d)];
    cnref_gemm_f32(1, 0, I, H, B, 1.f, x.data(), B, dt.data(), B, 1.f, gWih, I, nullptr, 0);
    cnref_gemm_f32(1, 0, H, H, B, 1.f, hp.data(), B, dt.data(), B, 1.f, gWhh, H, nullptr, 0);
    for (int64_t d = 0; d < H; ++d)
      for (int64_t n = 0; n < B; ++n) gb[d] += dt[(size_t)(n + B * d)];
    cnref_gemm_f32(0, 1, B, I, H, 1.f, dt.data(), B, Wih, I, 0.f, dx.data(), B, nullptr, 0);
    for (int64_t d = 0; d < I; ++d)
      for (int64_t n = 0; n < B; ++n) dX[n + B * t + B * S * d] = dx[(size_t)(n + B * d)];
    cnref_gemm_f32(0, 1, B, H, H, 1.f, dt.data(), B, Whh, H, 0.f, dh_next.data(), B, nullptr, 0);
  }
}

}  // extern "C"
