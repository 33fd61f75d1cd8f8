/*
 * cnref.h — CPU oracle for the CppNet "cpu-eigen" training semantics.
 *
 * TEST INFRASTRUCTURE ONLY.  This library restates, in plain C++17 loops,
 * what the reference computes on its "cpu-eigen" device (Eigen3 is absent
 * from this image, so the reference itself cannot be compiled here).  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it, and only as the checker or the timed CPU baseline; the product path
 * (cppnet_amd) never links, loads or calls it.
 *
 * Layout is Eigen ColMajor throughout (first index fastest), as in the
 * reference.  Every function cites the reference file:line it restates.
 * Sums run in ascending index order in fp32 unless stated otherwise; the
 * library is compiled without FMA contraction so each operation rounds once.
 */
#ifndef CNREF_H
#define CNREF_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

void cnref_set_threads(int n);
int  cnref_get_threads(void);
/* 1: GEMMs and the other reductions accumulate in double and round once,
 * and exp / log / tanh are evaluated in double and rounded once (another
 * valid evaluation of every rounding source, used to measure a trajectory's
 * sensitivity to rounding). */
void cnref_set_accumulate_double(int on);
/* The fp32 order of the GEMMs' k sums (when not double-accumulated):
 * 0 ascending k (default); 1 descending k; 2 chunks of 32 k summed from
 * zero, chunk sums added in order.  Three more valid evaluation orders,
 * used, like the double accumulation, to measure how far a trajectory
 * moves under rounding alone. */
void cnref_set_sum_order(int order);
/* 1: Linear forward and backward run as the reference's "cpu" device does
 * them (linear.cpp:196-215 forward_cpu, 289-330 backward_cpu: OpenMP over
 * the outputs, each output an fp32 sum over its contraction that the
 * compiler may vectorise), instead of the cpu-eigen contraction restated by
 * default.  Used to time the reference's "cpu" leg beside cpu-eigen. */
void cnref_set_cpu_loops(int on);
int  cnref_get_cpu_loops(void);

/* Optional diagnostic outputs for the tests' error bars (NULL = off).  While
 * a slot holds a buffer, the functions below also write:
 *   CNREF_TRACE_DPRE  recurrent backward (LSTM / GRU / RNN): the gradient of
 *                     every timestep's gate pre-activations, [B*S, G]
 *                     ColMajor (row n + B*t), G = 4H / 3H / H;
 *   CNREF_TRACE_GQP / _GKP / _GVP / _CTX   MHA backward: the gradients of
 *                     the three projections and the attention output
 *                     A*Vp of every sample, [B*S, D] (row n + B*s). */
#define CNREF_TRACE_DPRE 0
#define CNREF_TRACE_GQP 1
#define CNREF_TRACE_GKP 2
#define CNREF_TRACE_GVP 3
#define CNREF_TRACE_CTX 4
void cnref_set_trace(int slot, float* buf);
float* cnref_trace(int slot);

/* ColMajor C[M,N] = alpha*op(A)*op(B) + beta*C (+bias[n]) (relu if epi==1);
 * same operand conventions as cnhip_gemm_f32.  beta==0 does not read C. */
void cnref_gemm_f32(int ta, int tb, int64_t M, int64_t N, int64_t K, float alpha,
                    const float* A, int64_t lda, const float* B, int64_t ldb, float beta,
                    float* C, int64_t ldc, const float* bias, int epi);

/* Linear (linear.cpp:218-234 forward_eigen; 335-358 backward_eigen) */
void cnref_linear_forward(const float* X, const float* W, const float* b, float* Y,
                          int64_t B, int64_t I, int64_t O);
void cnref_linear_backward(const float* X, const float* W, const float* dY, float* gW,
                           float* gb, float* dX, int64_t B, int64_t I, int64_t O,
                           int trainable, int accumulate);
void cnref_column_sum(const float* in, float* out, int64_t rows, int64_t cols, int accumulate);

/* y = a + b elementwise (the cpu-eigen `out + shortcut` of residual.cpp:69-71
 * and `grad_block + grad_shortcut` of residual.cpp:113-115). */
void cnref_add(const float* a, const float* b, float* y, int64_t n);
/* Residual over [B, sizes[0]] (residual.cpp:44-159, cpu-eigen branches).
 * The block is n_block Linear layers, layer i mapping sizes[i] -> sizes[i+1]
 * with weights W[i] [sizes[i], sizes[i+1]] and bias b[i] (NULL: bias-free);
 * the shortcut is the input itself when Wp is NULL (then sizes[0] ==
 * sizes[n_block]) or the bias-free projection x Wp, Wp [sizes[0],
 * sizes[n_block]] (residual.cpp:31-36).
 * forward: acts[i] receives the output of block layer i ([B, sizes[i+1]];
 *   Linear::forward caches its input, so backward reads x and acts[0..n-2]);
 *   y = acts[n_block-1] + shortcut.
 * backward: the block's Linear backwards in reverse order, each accumulating
 *   into gW[i] / gb[i] (linear.cpp:346-352; gb[i] NULL when bias-free), the
 *   projection's backward on dY accumulating into gWp, and dX = the block's
 *   input gradient + the shortcut's (residual.cpp:89-131). */
void cnref_residual_forward(int n_block, const int64_t* sizes, const float* const* W,
                            const float* const* b, const float* Wp, const float* x,
                            float* const* acts, float* y, int64_t B);
void cnref_residual_backward(int n_block, const int64_t* sizes, const float* const* W,
                             const float* Wp, const float* x, const float* const* acts,
                             const float* dY, float* const* gW, float* const* gb, float* gWp,
                             float* dX, int64_t B);

/* Activations (relu.cpp:97-225; sigmoid.cpp:97-231; tanh.cpp:136-219) */
void cnref_relu_forward(const float* x, float* y, int64_t n);
void cnref_relu_backward(const float* y, const float* dy, float* dx, int64_t n);
void cnref_sigmoid_forward(const float* x, float* y, int64_t n);
void cnref_sigmoid_backward(const float* y, const float* dy, float* dx, int64_t n);
void cnref_tanh_forward(const float* x, float* y, int64_t n);
void cnref_tanh_backward(const float* y, const float* dy, float* dx, int64_t n);

/* Losses; reduction 0 = mean, 1 = sum */
float cnref_bce_forward(const float* p, const float* t, int64_t n, int reduction);
void  cnref_bce_backward(const float* p, const float* t, float* g, int64_t n, int reduction);
float cnref_mse_forward(const float* p, const float* t, int64_t n, int reduction);
void  cnref_mse_backward(const float* p, const float* t, float* g, int64_t n, int reduction);
float cnref_softmax_ce_forward(const float* z, const float* t, float* sm, int64_t B,
                               int64_t C, int reduction);
void  cnref_softmax_ce_backward(const float* sm, const float* t, float* g, int64_t B,
                                int64_t C, int reduction);

/* Conv2D, ColMajor X [N,C,H,W], W [OC,C,KS,KS], Y [N,OC,HO,WO] with
 * HO = (H + 2P - KS)/S + 1 (conv2d.cpp:78-136 forward; 138-198 backward:
 * grads OVERWRITE — zeroed, then accumulated over the batch).  b / gb may
 * be NULL (no bias).  dX is always computed. */
void cnref_conv2d_forward(const float* X, const float* W, const float* b, float* Y,
                          int64_t N, int64_t C, int64_t H, int64_t Wd, int64_t OC,
                          int64_t KS, int64_t S, int64_t P);
void cnref_conv2d_backward(const float* X, const float* W, const float* dY, float* gW,
                           float* gb, float* dX, int64_t N, int64_t C, int64_t H, int64_t Wd,
                           int64_t OC, int64_t KS, int64_t S, int64_t P);
/* MaxPool2D (max_pool2d.cpp:32-131): HO = (H - pool)/stride + 1, argmax is
 * the window-local ph*pool + pw of the first maximum (strict >, start -inf);
 * backward adds dY at the argmax of each window into a zeroed dX. */
void cnref_maxpool2d_forward(const float* X, float* Y, int32_t* idx, int64_t N, int64_t C,
                             int64_t H, int64_t W, int64_t pool, int64_t stride);
void cnref_maxpool2d_backward(const float* dY, const int32_t* idx, float* dX, int64_t N,
                              int64_t C, int64_t H, int64_t W, int64_t pool, int64_t stride);

/* LSTM (lstm.cpp:63-253).  X [B,S,I], Y [B,S,H] ColMajor; W_ih [I,4H],
 * W_hh [H,4H], b [4H] with gate column blocks i,f,g,o.  h0 = c0 = 0.
 * Forward caches, as [B*S, .] matrices (row n + B*t): gates = activations
 * i,f,g,o [B*S,4H], c [B*S,H], tanh_c [B*S,H].  Backward overwrites the
 * grads (lstm.cpp:158-160); dX may be NULL. */
void cnref_lstm_forward(const float* X, const float* Wih, const float* Whh, const float* b,
                        float* Y, float* gates, float* c, float* tanh_c, int64_t B, int64_t S,
                        int64_t I, int64_t H);
void cnref_lstm_backward(const float* X, const float* Wih, const float* Whh, const float* Y,
                         const float* gates, const float* c, const float* tanh_c,
                         const float* dY, float* gWih, float* gWhh, float* gb, float* dX,
                         int64_t B, int64_t S, int64_t I, int64_t H);
/* GRU (gru.cpp:56-315): gate blocks z,r,n of W_ih [I,3H], W_hh [H,3H],
 * b [3H]; n = tanh(x W_in + (r*h) W_hn + b_n); h = (1-z) n + z h_prev.
 * Caches: gates = z,r,n [B*S,3H], rh = r*h_prev [B*S,H]. */
void cnref_gru_forward(const float* X, const float* Wih, const float* Whh, const float* b,
                       float* Y, float* gates, float* rh, int64_t B, int64_t S, int64_t I,
                       int64_t H);
void cnref_gru_backward(const float* X, const float* Wih, const float* Whh, const float* Y,
                        const float* gates, const float* rh, const float* dY, float* gWih,
                        float* gWhh, float* gb, float* dX, int64_t B, int64_t S, int64_t I,
                        int64_t H);

/* Embedding (embedding.cpp:33-185): W [V,D] ColMajor, ids [B,S] int32,
 * out [B,S,D].  forward returns -1 (and writes nothing more) on an id out of
 * [0,V) (the cpu-eigen throw, 87-90); backward zeroes gW then adds. */
int  cnref_embedding_forward(const int32_t* ids, const float* W, float* out, int64_t B,
                             int64_t S, int64_t V, int64_t D);
void cnref_embedding_backward(const int32_t* ids, const float* dY, float* gW, int64_t B,
                              int64_t S, int64_t V, int64_t D);
/* MultiHeadAttention (attention.cpp:60-221 forward, 223-569 backward; the
 * cpu-eigen branches): per sample, Qp = Q Wq, Kp = K Wk, Vp = V Wv over the
 * full width D, A = softmax_rows(Qp Kp^T * 1/sqrt(D/heads)), out = (A Vp) Wo.
 * attn [B,S,S] ColMajor (n,i,j).  Grads overwrite; dX = dQ + dK + dV. */
void cnref_mha_forward(const float* q, const float* k, const float* v, const float* Wq,
                       const float* Wk, const float* Wv, const float* Wo, float* out,
                       float* attn, int64_t B, int64_t S, int64_t D, int64_t heads);
void cnref_mha_backward(const float* q, const float* k, const float* v, const float* Wq,
                        const float* Wk, const float* Wv, const float* Wo, const float* attn,
                        const float* dY, float* gWq, float* gWk, float* gWv, float* gWo,
                        float* dX, int64_t B, int64_t S, int64_t D, int64_t heads);
/* BatchNorm over x [N,F] (batch_norm.cpp:204-401), training mode: biased
 * batch variance, running stats (1-m) r + m batch. */
void cnref_batchnorm_forward(const float* x, float* y, float* xhat, const float* gamma,
                             const float* beta, float* running_mean, float* running_var,
                             float* batch_mean, float* batch_var, int64_t N, int64_t F,
                             float momentum, float eps);
void cnref_batchnorm_backward(const float* dY, const float* x, const float* xhat,
                              const float* gamma, const float* batch_mean,
                              const float* batch_var, float* ggamma, float* gbeta, float* dX,
                              int64_t N, int64_t F, float eps);
/* GELU, exact form x * Phi(x) = 0.5 x (1 + erf(x / sqrt 2)) (no reference:
 * the reference has no GELU); dX = dY (Phi(x) + x phi(x)). */
void cnref_gelu_forward(const float* x, float* y, int64_t n);
void cnref_gelu_backward(const float* x, const float* dy, float* dx, int64_t n);
/* MeanPool1D (mean_pool1d.cpp:24-150): [B,S,D] -> [B,D] mean over S;
 * backward dX = dY * (1/S). */
void cnref_meanpool1d_forward(const float* x, float* y, int64_t B, int64_t S, int64_t D);
void cnref_meanpool1d_backward(const float* dy, float* dx, int64_t B, int64_t S, int64_t D);

/* Adam, one tensor, caller-computed bias corrections (adam.cpp:98-133) */
void cnref_adam_step(float* W, const float* g, float* m, float* v, int64_t n, float lr,
                     float b1, float b2, float eps, float bc1, float bc2);
/* bias correction exactly as the reference: 1 - pow(beta, float(t)) in float */
float cnref_bias_correction(float beta, int t);

/* ---- cnref_extra.cpp: the reference's device ops off the BASELINE configs ---- */
void  cnref_leaky_relu_forward(const float* x, float* y, int64_t n, float alpha);
void  cnref_leaky_relu_backward(const float* x, const float* dy, float* dx, int64_t n, float alpha);
/* softmax over the last dimension: R rows, element (r, j) at r + R*j */
void  cnref_softmax_forward(const float* x, float* y, int64_t R, int64_t L);
void  cnref_softmax_backward(const float* y, const float* dy, float* dx, int64_t R, int64_t L);
float cnref_cce_forward(const float* pred, const float* t, float* sm, float* targets_used, int64_t B,
                        int64_t C, int from_logits, float label_smoothing, int reduction);
void  cnref_cce_backward(const float* sm, const float* targets_used, float* g, int64_t B, int64_t C,
                         int from_logits, int reduction);
float cnref_mae_forward(const float* p, const float* t, int64_t n, int reduction);
void  cnref_mae_backward(const float* p, const float* t, float* g, int64_t n, int reduction);
float cnref_huber_forward(const float* p, const float* t, int64_t n, float delta, int reduction);
void  cnref_huber_backward(const float* p, const float* t, float* g, int64_t n, float delta, int reduction);
void  cnref_sgd_step(float* W, const float* g, int64_t n, float lr);
void  cnref_momentum_step(float* W, const float* g, float* vel, int64_t n, float lr, float mu);
void  cnref_adagrad_step(float* W, const float* g, float* acc, int64_t n, float lr, float eps);
void  cnref_rmsprop_step(float* W, const float* g, float* s, int64_t n, float lr, float rho, float eps);
void  cnref_dropout_apply(const float* x, const float* mask, float* y, int64_t n, float scale);
void  cnref_global_avgpool_forward(const float* X, float* Y, int64_t N, int64_t C, int64_t H, int64_t W);
void  cnref_global_avgpool_backward(const float* dY, float* dX, int64_t N, int64_t C, int64_t H, int64_t W);
void  cnref_global_maxpool_forward(const float* X, float* Y, int32_t* ah, int32_t* aw, int64_t N,
                                   int64_t C, int64_t H, int64_t W);
void  cnref_global_maxpool_backward(const float* dY, const int32_t* ah, const int32_t* aw, float* dX,
                                    int64_t N, int64_t C, int64_t H, int64_t W);
void  cnref_rnn_forward(const float* X, const float* Wih, const float* Whh, const float* b, float* Y,
                        int64_t B, int64_t S, int64_t I, int64_t H);
void  cnref_rnn_backward(const float* X, const float* Wih, const float* Whh, const float* Y,
                         const float* dY, float* gWih, float* gWhh, float* gb, float* dX, int64_t B,
                         int64_t S, int64_t I, int64_t H);

#ifdef __cplusplus
}
#endif
#endif
