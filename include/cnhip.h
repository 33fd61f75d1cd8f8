/*
 * cnhip.h — C ABI of the MI355X (gfx950) training backend for CppNet.
 *
 * Every entry point takes device pointers, element counts / shapes and a
 * stream handle (NULL = the default stream), enqueues its kernels and returns
 * a status code.  Nothing here synchronises the device unless the comment
 * says so.  On a non-zero status, cnhip_last_error() returns a message that
 * names the entry point and the failed condition.
 *
 * Layout: every tensor is Eigen ColMajor, exactly as the reference stores it
 * (first index fastest):
 *   2-D [R,C]        (r,c)     -> r + R*c
 *   3-D [B,S,D]      (b,s,d)   -> b + B*(s + S*d)
 *   4-D [N,C,H,W]    (n,c,h,w) -> n + N*(c + C*(h + H*w))
 * so a [batch, features] matrix is batch-contiguous.
 *
 * Citations "ref: file:line" name the reference function (under
 * LoqmanSamani/CppNet) whose "gpu" branch the entry point replaces.
 */
#ifndef CNHIP_H
#define CNHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* cnhip_stream_t; /* a hipStream_t; NULL = default stream */

/* ---- status codes ------------------------------------------------------ */
#define CNHIP_OK              0
#define CNHIP_EINVAL          1  /* bad argument (shape, null pointer, enum) */
#define CNHIP_EHIP            2  /* HIP runtime error (launch, copy, device) */
#define CNHIP_ENOMEM          3  /* device allocation failed */
#define CNHIP_EUNSUPPORTED    4  /* valid but not supported here */

/* ---- runtime ----------------------------------------------------------- */
/* Message for the last non-zero status returned on this host thread. */
const char* cnhip_last_error(void);
/* Library version string, e.g. "cnhip 0.1 gfx950". */
const char* cnhip_version(void);
/* Number of visible HIP devices (0 when none); never fails. */
int cnhip_device_count(void);
/* Select the current device for this host thread. */
int cnhip_set_device(int device);
/* hipMalloc / hipFree / copies / fill; the runtime services the C++ host
 * layer uses (ref: the cudaMalloc/cudaMemcpy calls spread through every
 * "gpu" branch, e.g. src/CppNet/layers/linear.cpp:420-454). */
int cnhip_malloc(void** ptr, size_t bytes);
int cnhip_free(void* ptr);
/* kind: 0 host->device, 1 device->host, 2 device->device */
int cnhip_memcpy_async(void* dst, const void* src, size_t bytes, int kind,
                       cnhip_stream_t stream);
int cnhip_memset_async(void* dst, int value, size_t bytes, cnhip_stream_t stream);
int cnhip_stream_create(cnhip_stream_t* stream);
int cnhip_stream_destroy(cnhip_stream_t stream);
int cnhip_stream_synchronize(cnhip_stream_t stream);
int cnhip_device_synchronize(void);
/* 1 when ptr is device (or managed) memory of a HIP device, 0 otherwise. */
int cnhip_is_device_pointer(const void* ptr);
/* Events for timing on the stream the kernels run on. */
int cnhip_event_create(void** event);
int cnhip_event_destroy(void* event);
int cnhip_event_record(void* event, cnhip_stream_t stream);
int cnhip_event_elapsed_ms(float* ms, void* start, void* stop); /* syncs stop */
int cnhip_event_synchronize(void* event);
/* Work enqueued on stream after this call waits for event's work. */
int cnhip_stream_wait_event(cnhip_stream_t stream, void* event);
int cnhip_get_device(int* device);
/* Page-locked host memory (hipHostMalloc), for asynchronous uploads. */
int cnhip_host_alloc(void** ptr, size_t bytes);
int cnhip_host_free(void* ptr);
/* cnhip_memset_async fills with a kernel, so it can be recorded into a graph. */

/* ---- graphs -------------------------------------------------------------
 * Capture of the work enqueued on one created stream into a HIP graph, and
 * its replay.  No counterpart in the reference (its "gpu" branches copy
 * host<->device inside every call and cannot be captured); this replaces
 * the per-kernel launch cost of a whole training step with one graph launch.
 *   begin_capture: starts capturing `stream` (relaxed mode; refused while
 *     per-launch GEMM timing is on).  Nothing enqueued on it runs until the
 *     graph is launched.
 *   end_capture: ends the capture; with ok != 0 instantiates the graph into
 *     *graph, with ok == 0 discards it (*graph = NULL).  While a graph
 *     exists, the stream's scratch slots are frozen: work that would need a
 *     larger scratch buffer on that stream fails with CNHIP_EUNSUPPORTED
 *     instead of moving the buffer the graph refers to.  So run the work
 *     once uncaptured (at the same shapes) before capturing it.
 *   launch: replays the graph on the stream it was captured on.
 *   destroy: synchronises that stream, frees the graph, unfreezes. */
typedef void* cnhip_graph_t;
int cnhip_graph_begin_capture(cnhip_stream_t stream);
int cnhip_graph_end_capture(cnhip_stream_t stream, int ok, cnhip_graph_t* graph);
int cnhip_graph_launch(cnhip_graph_t graph, cnhip_stream_t stream);
int cnhip_graph_destroy(cnhip_graph_t graph);

/* ---- GEMM ---------------------------------------------------------------
 * ColMajor  C[M,N] = alpha * op(A)[M,K] * op(B)[K,N] + beta * C  (+ bias[n])
 *   trans_a == 0: A(m,k) = A[m + lda*k];  trans_a == 1: A(m,k) = A[k + lda*m]
 *   trans_b == 0: B(k,n) = B[k + ldb*n];  trans_b == 1: B(k,n) = B[n + ldb*k]
 * beta == 0 never reads C.  bias may be NULL.  epilogue: 0 none, 1 ReLU
 * applied after bias.  fp32 in, fp32 MFMA (v_mfma_f32_32x32x2f32), fp32 out.
 * ref: src/CppNet/kernels/gpu/matmul.cu:16-71 (NN), matmul_grad_input.cu:14-68
 * (NT), matmul_grad_weight.cu:14-69 (TN), add_bias.cu:13-22 (bias epilogue). */
#define CNHIP_EPI_NONE 0
#define CNHIP_EPI_RELU 1
int cnhip_gemm_f32(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K,
                   float alpha, const float* A, int64_t lda,
                   const float* B, int64_t ldb, float beta,
                   float* C, int64_t ldc, const float* bias, int epilogue,
                   cnhip_stream_t stream);

/* Strided-batched form: for b in [0, batch_count): the GEMM above on
 * A + b*stride_a, B + b*stride_b, C + b*stride_c (no bias, no epilogue).
 * Used for per-timestep / per-sample products (LSTM, attention).
 * ref: the per-sample contractions of attention.cpp:183-212 and the
 * per-timestep ones of lstm.cpp:104-105, 228-244. */
int cnhip_gemm_f32_batched(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K,
                           float alpha, const float* A, int64_t lda, int64_t stride_a,
                           const float* B, int64_t ldb, int64_t stride_b, float beta,
                           float* C, int64_t ldc, int64_t stride_c, int64_t batch_count,
                           cnhip_stream_t stream);


/* Measurement aid for the MFMA GEMM-shaped kernels (the GEMM kernel and the
 * implicit-GEMM Conv2D forward / dgrad / wgrad kernels): while enabled,
 * every such launch on this host thread is bracketed by HIP events on its
 * own stream, and its algorithmic flops (2*M*N*K; for Conv2D
 * 2*N*HO*WO*OC*C*KS^2) recorded.
 * read() synchronises those events and returns the launch count, the summed
 * kernel time (ms) and the summed flops since the last enable(1).  Split-K
 * reduction launches are not counted.  Not a reference function. */
int cnhip_gemm_timing_enable(int on);
int cnhip_gemm_timing_read(int64_t* launches, double* total_ms, double* total_flops);
/* Per-launch timing of the bandwidth-bound kernels (elementwise, reductions,
 * pooling, normalisation, transposes, Adam, split-K reduces): while on, each
 * such launch is bracketed by events on its stream and credited with its
 * algorithmic HBM bytes (each input read once, each output written once).
 * read() aggregates per kernel name, in first-seen order, into rows[0 ..
 * max_rows) and sets *n_rows to the number of kernels seen (which may exceed
 * max_rows); it synchronises on the recorded events.  No counterpart in the
 * reference: this is the measurement the BASELINE metric asks of
 * bandwidth-bound kernels. */
typedef struct {
  const char* kernel;   /* kernel name (static string of the library) */
  int64_t launches;
  double total_ms;      /* sum of the launches' event-timed durations */
  double total_bytes;   /* sum of their algorithmic HBM bytes */
} cnhip_kernel_timing;
int cnhip_hbm_timing_enable(int on);
int cnhip_hbm_timing_read(cnhip_kernel_timing* rows, int max_rows, int* n_rows);

/* ---- Linear ------------------------------------------------------------ */
/* Y[B,O] = X[B,I] * W[I,O] + b[O]   (b may be NULL)
 * ref: Linear::forward_gpu, src/CppNet/layers/linear.cpp:456-500 */
int cnhip_linear_forward(const float* X, const float* W, const float* b,
                         float* Y, int64_t batch, int64_t in_features,
                         int64_t out_features, cnhip_stream_t stream);
/* grad_W[I,O] += X^T dY ; grad_b[O] += colsum(dY)   (when trainable; grad_b
 * skipped when NULL) ; dX[B,I] = dY W^T (skipped when dX is NULL).
 * accumulate: 1 adds into grad_W/grad_b (the cpu-eigen semantics,
 * linear.cpp:346-352), 0 overwrites them.
 * ref: Linear::backward_gpu, src/CppNet/layers/linear.cpp:502-539 and
 * Linear::backward_eigen, linear.cpp:335-358 */
int cnhip_linear_backward(const float* X, const float* W, const float* dY,
                          float* grad_W, float* grad_b, float* dX,
                          int64_t batch, int64_t in_features,
                          int64_t out_features, int trainable, int accumulate,
                          cnhip_stream_t stream);
/* Linear fused with the activation that follows it (the producing GEMM's
 * epilogue applies it; no separate elementwise pass):
 *   act CNHIP_ACT_RELU: Y = max(X W + b, 0)               (Z unused, may be NULL)
 *   act CNHIP_ACT_GELU: Z = X W + b, Y = Z Phi(Z)         (Z is GELU's backward input)
 * and the matching backward, whose dX GEMM applies the derivative of the
 * activation on the layer BELOW (the one that produced this layer's input):
 *   dX = (dY W^T) * [act_aux > 0]   (RELU: act_aux = that ReLU's output)
 *   dX = (dY W^T) * gelu'(act_aux)  (GELU: act_aux = that GELU's input Z)
 * CNHIP_ACT_RESIDUAL fuses a skip connection instead of an activation:
 *   forward  Y = (X W + b) + Z          (Z read: the skip branch, [B,O])
 *   backward dX = dY W^T + act_aux      (act_aux: the skip branch's gradient, [B,I])
 * Weight/bias grads as cnhip_linear_backward.  Results equal the unfused
 * layer + activation (or add) calls: same arithmetic per element.
 * ref: Linear::forward/backward (linear.cpp:148-358) chained with
 * ReLU::forward/backward (relu.cpp:97-225), or with the residual sum of
 * Residual::forward/backward (residual.cpp:44-159); GELU has no reference. */
#define CNHIP_ACT_NONE 0
#define CNHIP_ACT_RELU 1
#define CNHIP_ACT_GELU 2
#define CNHIP_ACT_RESIDUAL 3
int cnhip_linear_forward_act(const float* X, const float* W, const float* b, float* Y,
                             float* Z, int64_t batch, int64_t in_features,
                             int64_t out_features, int act, cnhip_stream_t stream);
int cnhip_linear_backward_act(const float* X, const float* W, const float* dY,
                              float* grad_W, float* grad_b, float* dX, const float* act_aux,
                              int64_t batch, int64_t in_features, int64_t out_features,
                              int trainable, int accumulate, int act, cnhip_stream_t stream);
/* cnhip_linear_backward_act for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Same arguments, kernels and
 * results, bit for bit; it calls no hipMalloc / hipFree and creates no
 * events.  The kernels' workspace (split-K partials, the one-pass head's
 * row-chunk partials) is a fixed 32 MiB device array per GPU, looked up on
 * the first call on each device; a shape that would need more is refused
 * with CNHIP_EINVAL before anything runs.  Nothing in the workspace has to
 * start at zero.  Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (two streams, or two host threads) race. */
int cnhip_linear_backward_act_noalloc(const float* X, const float* W, const float* dY,
                                      float* grad_W, float* grad_b, float* dX,
                                      const float* act_aux, int64_t batch, int64_t in_features,
                                      int64_t out_features, int trainable, int accumulate,
                                      int act, cnhip_stream_t stream);
/* out[j] (+)= sum_r in[r + rows*j]   — column sums of a ColMajor [rows,cols]
 * ref: src/CppNet/kernels/gpu/bias_grad.cu:12-46 */
int cnhip_column_sum(const float* in, float* out, int64_t rows, int64_t cols,
                     int accumulate, cnhip_stream_t stream);

/* ---- Conv2D / MaxPool2D / Flatten ----------------------------------------
 * X [N,C,H,W], W [OC,C,KS,KS], Y [N,OC,HO,WO], HO = (H + 2P - KS)/S + 1.
 * backward OVERWRITES grad_W / grad_b (the reference zeroes them first,
 * conv2d.cpp:149-152); b / grad_b / dX may be NULL.
 * ref: Conv2D::forward/backward src/CppNet/layers/conv2d.cpp:78-198;
 * conv2d_forward.cu:16-64, conv2d_backward.cu:19-68 */
int cnhip_conv2d_forward(const float* X, const float* W, const float* b, float* Y,
                         int64_t N, int64_t C, int64_t H, int64_t Wd, int64_t OC,
                         int64_t KS, int64_t S, int64_t P, cnhip_stream_t stream);
/* Conv2D forward followed by ReLU: Y = max(0, conv(X) + b), bit-identical to
 * cnhip_conv2d_forward then cnhip_relu_forward.  Replaces the pair
 * Conv2D::forward (conv2d.cpp:78-130) + the 4-D ReLU::forward (relu.cpp:
 * 128-160) of a Conv2D -> ReLU stack; Y is the ReLU output the ReLU's
 * backward reads. */
int cnhip_conv2d_forward_relu(const float* X, const float* W, const float* b, float* Y,
                              int64_t N, int64_t C, int64_t H, int64_t Wd, int64_t OC,
                              int64_t KS, int64_t S, int64_t P, cnhip_stream_t stream);
/* Conv2D forward, ReLU and MaxPool2D in one call: Yp = maxpool(max(0,
 * conv(X) + b)) [N,OC,HP,WP] and idx its int32 argmax, bit-identical to
 * cnhip_conv2d_forward_relu then cnhip_maxpool2d_forward (pool_stride <= 0
 * means pool).  The ReLU output is not kept: the pool's backward takes its
 * mask from Yp (cnhip_maxpool2d_backward_relu_pooled).  Replaces the three
 * forwards Conv2D::forward (conv2d.cpp:78-130), the 4-D ReLU::forward
 * (relu.cpp:128-160) and MaxPool2D::forward (max_pool2d.cpp:32-95) of a
 * Conv2D -> ReLU -> MaxPool2D stack.  One kernel for short contractions
 * (C*KS*KS <= 32, OC % 32 == 0, N % 64 == 0, pool_stride == pool <= 4
 * tiling the conv output), otherwise the two steps through a workspace. */
int cnhip_conv2d_forward_relu_maxpool(const float* X, const float* W, const float* b, float* Yp,
                                      int32_t* idx, int64_t N, int64_t C, int64_t H, int64_t Wd,
                                      int64_t OC, int64_t KS, int64_t S, int64_t P, int64_t pool,
                                      int64_t pool_stride, cnhip_stream_t stream);
int cnhip_conv2d_backward(const float* X, const float* W, const float* dY,
                          float* grad_W, float* grad_b, float* dX, int64_t N, int64_t C,
                          int64_t H, int64_t Wd, int64_t OC, int64_t KS, int64_t S,
                          int64_t P, cnhip_stream_t stream);
/* The weight and bias gradients of a Conv2D -> ReLU -> MaxPool2D stack whose
 * forward ran as cnhip_conv2d_forward_relu_maxpool, straight from the pooled
 * gradient dP [N,OC,HP,WP], the argmax idx and the pooled output Pout: the
 * gradient at the conv output is formed while the weight-gradient GEMM loads
 * it (routed to each window's argmax, masked by Pout > 0, as
 * cnhip_maxpool2d_backward_relu_pooled writes it) and never stored, so
 * grad_W and grad_b (overwritten) equal that call followed by
 * cnhip_conv2d_backward bit for bit.  No input gradient: for a model's first
 * layer, whose input is data.  Takes pool windows tiling the conv output
 * (pool_stride == pool, or <= 0), N % 64 == 0 and 16-byte aligned X, dP, idx,
 * Pout (cnhip_conv2d_backward_maxpool_relu_fits: 1 when the shape fits).
 * Replaces Conv2D::backward (conv2d.cpp:131-198, weight and bias part),
 * ReLU::backward (relu.cpp:194-225) and MaxPool2D::backward
 * (max_pool2d.cpp:96-131) of that stack. */
int cnhip_conv2d_backward_maxpool_relu(const float* X, const float* dP, const int32_t* idx,
                                       const float* Pout, float* grad_W, float* grad_b, int64_t N,
                                       int64_t C, int64_t H, int64_t Wd, int64_t OC, int64_t KS,
                                       int64_t S, int64_t P, int64_t pool, int64_t pool_stride,
                                       cnhip_stream_t stream);
int cnhip_conv2d_backward_maxpool_relu_fits(int64_t N, int64_t C, int64_t H, int64_t Wd, int64_t OC,
                                            int64_t KS, int64_t S, int64_t P, int64_t pool,
                                            int64_t pool_stride);
/* MaxPool2D: Y [N,C,HO,WO], HO = (H - pool)/stride + 1 (stride <= 0 means
 * pool); idx = int32 window-local ph*pool + pw of the first maximum;
 * backward writes every element of dX (no pre-zeroing needed).
 * ref: MaxPool2D::forward/backward max_pool2d.cpp:32-131;
 * maxpool2d_forward.cu:17-59, maxpool2d_backward.cu:16-46.
 * Flatten (flatten.cpp:15-39) is a ColMajor reshape: no kernel. */
int cnhip_maxpool2d_forward(const float* X, float* Y, int32_t* idx, int64_t N, int64_t C,
                            int64_t H, int64_t W, int64_t pool, int64_t stride,
                            cnhip_stream_t stream);
int cnhip_maxpool2d_backward(const float* dY, const int32_t* idx, float* dX, int64_t N,
                             int64_t C, int64_t H, int64_t W, int64_t pool, int64_t stride,
                             cnhip_stream_t stream);
/* MaxPool2D backward followed by the backward of the ReLU that produced the
 * pool's input y (= the ReLU output, [N,C,H,W]): dX = maxpool_backward(dY) *
 * [y > 0], bit-identical to cnhip_maxpool2d_backward then cnhip_relu_backward.
 * Replaces the pair MaxPool2D::backward (max_pool2d.cpp:96-131) + the 4-D
 * ReLU::backward (relu.cpp:194-225) that a Conv2D -> ReLU -> MaxPool2D stack
 * runs. */
int cnhip_maxpool2d_backward_relu(const float* dY, const int32_t* idx, const float* y, float* dX,
                                  int64_t N, int64_t C, int64_t H, int64_t W, int64_t pool,
                                  int64_t stride, cnhip_stream_t stream);
/* The same with the ReLU mask taken from the pool's output Y [N,C,HO,WO]
 * (whose value at a window is the ReLU output at its argmax): dX equals
 * cnhip_maxpool2d_backward_relu's (bit for bit when the windows tile the
 * input; where overlapping windows add several terms the masked ones are
 * zeros).  For the output of cnhip_conv2d_forward_relu_maxpool.
 * ref: as cnhip_maxpool2d_backward_relu. */
int cnhip_maxpool2d_backward_relu_pooled(const float* dY, const int32_t* idx, const float* Y, float* dX,
                                         int64_t N, int64_t C, int64_t H, int64_t W, int64_t pool,
                                         int64_t stride, cnhip_stream_t stream);
/* Backward of a classifier head Conv2D -> ReLU -> MaxPool2D -> Flatten ->
 * Linear(F -> O) from the Linear's output gradient dZ [N, O] to the ReLU's
 * input, in one pass: grad_W [F, O] (+)= P^T dZ and grad_b (+)= the column
 * sums of dZ (accumulate as cnhip_linear_backward), and dX [N, C, H, W] =
 * the pool's backward of (dZ W^T) with the ReLU mask from P, as
 * cnhip_linear_backward then cnhip_maxpool2d_backward_relu_pooled compute
 * them.  P [N, C, HO, WO] is the pooled output (the Linear's input, F =
 * C HO WO) and idx its argmax, as cnhip_conv2d_forward_relu_maxpool writes
 * them.  Sums run in a fixed order (a lane's rows, then an xor butterfly
 * over the lanes; dX over O ascending), so the results can differ from
 * the separate calls' in the last bits.  Needs
 * windows that tile the input (stride == pool, dividing H and W), O <= 16
 * and N O <= 8192 (cnhip_linear_backward_maxpool_relu_fits).  Replaces
 * Linear::backward (linear.cpp:335-358) + Flatten::backward + MaxPool2D::
 * backward (max_pool2d.cpp:96-131) + ReLU::backward (relu.cpp:194-225). */
int cnhip_linear_backward_maxpool_relu(const float* P, const int32_t* idx, const float* W, const float* dZ,
                                       float* grad_W, float* grad_b, float* dX, int64_t N, int64_t C,
                                       int64_t H, int64_t Wd, int64_t out_features, int64_t pool,
                                       int64_t stride, int accumulate, cnhip_stream_t stream);
int cnhip_linear_backward_maxpool_relu_fits(int64_t N, int64_t C, int64_t H, int64_t W,
                                            int64_t out_features, int64_t pool, int64_t stride);

/* ---- recurrent layers ----------------------------------------------------
 * X [B,S,I], Y [B,S,H] ColMajor (row n + B*t of a [B*S, .] matrix).
 * LSTM: W_ih [I,4H], W_hh [H,4H], b [4H], gate blocks i,f,g,o; h0 = c0 = 0.
 * forward writes Y and the caches gates (activations, [B*S,4H]), c and
 * tanh_c ([B*S,H]); backward reads them and OVERWRITES the grads
 * (lstm.cpp:158-160); dX may be NULL.
 * ref: LSTM::forward/backward src/CppNet/layers/lstm.cpp:63-253;
 * lstm_cell.cu:21-114 */
/* Faults of the persistent recurrence.  The LSTM recurrence runs as one
 * launch per pass whose blocks wait for each other's values every step;
 * every wait is bounded, and a launch that gives up leaves invalid outputs
 * and sets a device guard: until the fault is taken, every optimizer launch
 * on the device (cnhip_adam_step[_multi], cnhip_optimizer_step_multi)
 * leaves its tensors unchanged, so the invalid values never reach the
 * parameters.  cnhip_recurrence_fault_check returns CNHIP_OK when no fault
 * is pending (one read of a pinned host word); otherwise it takes the fault
 * (synchronizes the device, clears the guard) and returns CNHIP_EHIP.  The
 * recurrent calls and cnhip_graph_launch check on entry; a caller that
 * synchronizes (a loss read-back) checks after it.  Each optimizer launch
 * gets a sequence number, increasing over the process
 * (cnhip_update_seq_last: this thread's last one); cnhip_update_withheld(seq)
 * is 1 when that launch (on the current device) was withheld by a fault
 * taken so far, and cnhip_update_faults_taken counts those faults, so a
 * caller can roll back the step counts of its withheld updates.  No
 * counterpart in the reference (its recurrence is a host loop). */
int cnhip_recurrence_fault_check(cnhip_stream_t stream);
/* Measurement aid for the persistent LSTM kernels (no reference
 * counterpart): while set, every persistent forward (backward) launch whose
 * (B/16) (H/16) S 8 entries fit `capacity` records, per block and timestep,
 * a 100 MHz realtime counter at its phase boundaries into fwd (bwd), a
 * device array of uint64 [blocks][S][8] (block = sample tile H/16 + unit
 * tile); forward phases: step start, h_{t-1} arrived, vote, gates, step
 * end; backward: step start, weight-gradient MFMAs done, partials arrived,
 * vote, cell backward done, partials handed on.  NULL / 0 switches it off.
 * The buffers must outlive the launches that use them. */
int cnhip_lstm_phase_stamps(uint64_t* fwd, uint64_t* bwd, int64_t capacity);
int64_t cnhip_update_seq_last(void);
int64_t cnhip_update_faults_taken(void);
int cnhip_update_withheld(int64_t seq);
int cnhip_lstm_forward(const float* X, const float* W_ih, const float* W_hh, const float* b,
                       float* Y, float* gates, float* c, float* tanh_c, int64_t B, int64_t S,
                       int64_t I, int64_t H, cnhip_stream_t stream);
int cnhip_lstm_backward(const float* X, const float* W_ih, const float* W_hh, const float* Y,
                        const float* gates, const float* c, const float* tanh_c,
                        const float* dY, float* grad_W_ih, float* grad_W_hh, float* grad_b,
                        float* dX, int64_t B, int64_t S, int64_t I, int64_t H,
                        cnhip_stream_t stream);
/* cnhip_lstm_backward for a gradient that reaches only the last step's
 * output: dY_last [B,H] is dY at t = S-1, dY being 0 at every other step.
 * Results equal cnhip_lstm_backward on that dY.  Replaces the spread of the
 * gradient over [B,S,H] (the backward of taking the last step,
 * cnhip_seq_scatter) plus the LSTM backward (lstm.cpp:184-253) of an
 * LSTM -> last step -> Linear model. */
int cnhip_lstm_backward_last(const float* X, const float* W_ih, const float* W_hh, const float* Y,
                             const float* gates, const float* c, const float* tanh_c,
                             const float* dY_last, float* grad_W_ih, float* grad_W_hh, float* grad_b,
                             float* dX, int64_t B, int64_t S, int64_t I, int64_t H,
                             cnhip_stream_t stream);
/* GRU: W_ih [I,3H], W_hh [H,3H], b [3H], gate blocks z,r,n with
 * n = tanh(x W_in + (r*h) W_hn + b_n), h = (1-z) n + z h_prev; caches gates
 * (z,r,n activations [B*S,3H]) and rh = r*h_prev [B*S,H].
 * ref: GRU::forward/backward src/CppNet/layers/gru.cpp:56-297; gru_cell.cu:20-140 */
int cnhip_gru_forward(const float* X, const float* W_ih, const float* W_hh, const float* b,
                      float* Y, float* gates, float* rh, int64_t B, int64_t S, int64_t I,
                      int64_t H, cnhip_stream_t stream);
int cnhip_gru_backward(const float* X, const float* W_ih, const float* W_hh, const float* Y,
                       const float* gates, const float* rh, const float* dY, float* grad_W_ih,
                       float* grad_W_hh, float* grad_b, float* dX, int64_t B, int64_t S,
                       int64_t I, int64_t H, cnhip_stream_t stream);
/* out[B,D] = Y[:, t, :]; and Y = 0 except Y[:, t, :] = in.  The harness's
 * last-hidden-state slice and its gradient (sequence_benckmark.cpp:152-170). */
int cnhip_seq_select(const float* Y, float* out, int64_t B, int64_t S, int64_t D, int64_t t,
                     cnhip_stream_t stream);
int cnhip_seq_scatter(const float* in, float* Y, int64_t B, int64_t S, int64_t D, int64_t t,
                      cnhip_stream_t stream);

/* ---- transformer layers ----------------------------------------------------
 * Sequences [B,S,D] are ColMajor (row b + B*s of a [B*S, D] matrix).
 *
 * Row order.  The `_rows` variants also take CNHIP_ROWS_BY_SAMPLE: every
 * [B*S, D] sequence argument then holds row s + S*b (sample b's S rows
 * adjacent), which is what the batched attention products read without
 * transposing; ids stay ColMajor [B, S] and pooled outputs [B, D].  These
 * variants have no reference counterpart: the reference has one row order.
 * They are for a caller that owns the whole Embedding -> MeanPool1D chain,
 * so that the order never reaches its user. */
#define CNHIP_ROWS_REF 0       /* row b + B*s (the reference's [B,S,D]) */
#define CNHIP_ROWS_BY_SAMPLE 1 /* row s + S*b */

/* out [cols, rows] = in [rows, cols]^T, both ColMajor. */
int cnhip_transpose(const float* in, float* out, int64_t rows, int64_t cols,
                    cnhip_stream_t stream);
/* MultiHeadAttention: one full-width head, scale 1/sqrt(D/heads), no biases;
 * out = softmax_rows(Q Wq (K Wk)^T * scale) (V Wv) Wo per sample.  forward
 * fills `cache` (cnhip_mha_cache_floats(B,S,D) floats: the projections and
 * attention weights backward reads); backward OVERWRITES the four weight
 * grads and writes dX = dQ + dK + dV (dX may be NULL).  When q == k == v and
 * Wq, Wk, Wv (and gWq, gWk, gWv) are adjacent D*D blocks, the three
 * projections run as one GEMM.
 * ref: MultiHeadAttention::forward/backward
 * src/CppNet/layers/attention.cpp:60-221, 503-569 (cpu-eigen branches) */
int64_t cnhip_mha_cache_floats(int64_t B, int64_t S, int64_t D);
int cnhip_mha_forward(const float* q, const float* k, const float* v, const float* Wq,
                      const float* Wk, const float* Wv, const float* Wo, float* out,
                      float* cache, int64_t B, int64_t S, int64_t D, int64_t heads,
                      cnhip_stream_t stream);
int cnhip_mha_backward(const float* q, const float* k, const float* v, const float* Wq,
                       const float* Wk, const float* Wv, const float* Wo, const float* cache,
                       const float* dY, float* gWq, float* gWk, float* gWv, float* gWo,
                       float* dX, int64_t B, int64_t S, int64_t D, int64_t heads,
                       cnhip_stream_t stream);
/* The same with a skip connection fused into the last GEMM of each pass:
 * forward out = MHA(q, k, v) + residual; backward dX = dQ + dK + dV +
 * residual_grad (dX required).  Equal to the unfused call followed by
 * cnhip_add.  ref: MultiHeadAttention::forward/backward (attention.cpp:60-221,
 * 503-569) followed by a skip sum F(x) + x as Residual::forward/backward
 * computes it (residual.cpp:44-159). */
int cnhip_mha_forward_residual(const float* q, const float* k, const float* v, const float* Wq,
                               const float* Wk, const float* Wv, const float* Wo,
                               const float* residual, float* out, float* cache, int64_t B,
                               int64_t S, int64_t D, int64_t heads, cnhip_stream_t stream);
int cnhip_mha_backward_residual(const float* q, const float* k, const float* v, const float* Wq,
                                const float* Wk, const float* Wv, const float* Wo,
                                const float* cache, const float* dY, const float* residual_grad,
                                float* gWq, float* gWk, float* gWv, float* gWo, float* dX,
                                int64_t B, int64_t S, int64_t D, int64_t heads,
                                cnhip_stream_t stream);
/* cnhip_mha_forward_residual / _backward_residual in either row order
 * (residual / residual_grad may be NULL: the unfused pass). */
int cnhip_mha_forward_rows(const float* q, const float* k, const float* v, const float* Wq,
                           const float* Wk, const float* Wv, const float* Wo,
                           const float* residual, float* out, float* cache, int64_t B,
                           int64_t S, int64_t D, int64_t heads, int rows,
                           cnhip_stream_t stream);
int cnhip_mha_backward_rows(const float* q, const float* k, const float* v, const float* Wq,
                            const float* Wk, const float* Wv, const float* Wo,
                            const float* cache, const float* dY, const float* residual_grad,
                            float* gWq, float* gWk, float* gWv, float* gWo, float* dX,
                            int64_t B, int64_t S, int64_t D, int64_t heads, int rows,
                            cnhip_stream_t stream);
/* Embedding: weights kept token-major, Wt[d + D*v] (the transpose of the
 * reference's ColMajor [V, D]); ids [B,S] int32; out [B,S,D].  Ids outside
 * [0, V) give zero rows and are counted into *oob_count (may be NULL; the
 * host layer checks it and raises, as the cpu-eigen branch throws).
 * backward OVERWRITES gWt (rows of unused ids become 0) with a deterministic
 * per-token sum in position order.
 * ref: Embedding::forward/backward src/CppNet/layers/embedding.cpp:46-175;
 * embedding_forward.cu, embedding_backward.cu */
int cnhip_embedding_forward(const int32_t* ids, const float* Wt, float* out, int64_t B,
                            int64_t S, int64_t V, int64_t D, int32_t* oob_count,
                            cnhip_stream_t stream);
int cnhip_embedding_backward(const int32_t* ids, const float* dY, float* gWt, int64_t B,
                             int64_t S, int64_t V, int64_t D, cnhip_stream_t stream);
/* the same in either row order (of out and dY) */
int cnhip_embedding_forward_rows(const int32_t* ids, const float* Wt, float* out, int64_t B,
                                 int64_t S, int64_t V, int64_t D, int32_t* oob_count, int rows,
                                 cnhip_stream_t stream);
int cnhip_embedding_backward_rows(const int32_t* ids, const float* dY, float* gWt, int64_t B,
                                  int64_t S, int64_t V, int64_t D, int rows,
                                  cnhip_stream_t stream);
/* BatchNorm over x [N,F] in training mode: biased batch variance,
 * xhat = (x - mean)/sqrt(var + eps), y = gamma xhat + beta, running stats
 * (1-momentum) r + momentum * batch.  backward OVERWRITES grad_gamma and
 * grad_beta.  xhat may be NULL in both: the forward then does not store it
 * and the backward recomputes it from x, batch_mean and batch_var with the
 * forward's exact expression (bit-identical), 8 + 12 instead of 12 + 16
 * bytes per element; pass the cached xhat to the backward after an
 * eval-mode forward (the reference's backward reads its cached x_hat_).
 * ref: BatchNorm::forward/backward
 * src/CppNet/layers/batch_norm.cpp:204-401; batch_norm_forward.cu,
 * batch_norm_backward.cu */
int cnhip_batchnorm_forward(const float* x, float* y, float* xhat, const float* gamma,
                            const float* beta, float* running_mean, float* running_var,
                            float* batch_mean, float* batch_var, int64_t N, int64_t F,
                            float momentum, float eps, cnhip_stream_t stream);
/* eval mode: xhat = (x - running_mean)/sqrt(running_var + eps)
 * (batch_norm.cpp:320-327); statistics untouched. */
int cnhip_batchnorm_forward_eval(const float* x, float* y, float* xhat, const float* gamma,
                                 const float* beta, const float* running_mean,
                                 const float* running_var, int64_t N, int64_t F, float eps,
                                 cnhip_stream_t stream);
int cnhip_batchnorm_backward(const float* dY, const float* x, const float* xhat,
                             const float* gamma, const float* batch_mean,
                             const float* batch_var, float* grad_gamma, float* grad_beta,
                             float* dX, int64_t N, int64_t F, float eps, cnhip_stream_t stream);
/* GELU, exact form y = x Phi(x) = 0.5 x (1 + erf(x/sqrt 2)); dx = dy (Phi(x)
 * + x phi(x)).  No reference counterpart: the reference has no GELU. */
int cnhip_gelu_forward(const float* x, float* y, int64_t n, cnhip_stream_t stream);
int cnhip_gelu_backward(const float* x, const float* dy, float* dx, int64_t n,
                        cnhip_stream_t stream);
/* MeanPool1D: y [B,D] = mean over s of x [B,S,D]; dx = dy / S broadcast.
 * ref: MeanPool1D::forward/backward src/CppNet/layers/mean_pool1d.cpp:24-150;
 * mean_pool1d.cu:27-69 */
int cnhip_meanpool1d_forward(const float* x, float* y, int64_t B, int64_t S, int64_t D,
                             cnhip_stream_t stream);
int cnhip_meanpool1d_backward(const float* dy, float* dx, int64_t B, int64_t S, int64_t D,
                              cnhip_stream_t stream);
/* the same in either row order (of x and dx) */
int cnhip_meanpool1d_forward_rows(const float* x, float* y, int64_t B, int64_t S, int64_t D,
                                  int rows, cnhip_stream_t stream);
int cnhip_meanpool1d_backward_rows(const float* dy, float* dx, int64_t B, int64_t S, int64_t D,
                                   int rows, cnhip_stream_t stream);
/* y = a + b (the residual add and its gradient sum).
 * ref: Residual::forward/backward src/CppNet/layers/residual.cpp:44-159 */
int cnhip_add(const float* a, const float* b, float* y, int64_t n, cnhip_stream_t stream);

/* ---- activations (elementwise over n values) -------------------------- */
/* ReLU: y = max(x,0); dx = dy * (y > 0)   (mask from the cached OUTPUT)
 * ref: relu.cu:14-23, relu_grad.cu:11-19; ReLU::forward/backward
 * src/CppNet/activations/relu.cpp:97-225 */
int cnhip_relu_forward(const float* x, float* y, int64_t n, cnhip_stream_t stream);
int cnhip_relu_backward(const float* y, const float* dy, float* dx, int64_t n,
                        cnhip_stream_t stream);
/* Sigmoid: y = 1/(1+exp(-clamp(x,-500,500))); dx = dy*y*(1-y)
 * ref: sigmoid.cu:13-23, sigmoid_grad.cu:11-20; sigmoid.cpp:97-231 */
int cnhip_sigmoid_forward(const float* x, float* y, int64_t n, cnhip_stream_t stream);
int cnhip_sigmoid_backward(const float* y, const float* dy, float* dx, int64_t n,
                           cnhip_stream_t stream);
/* Tanh: y = tanh(x); dx = dy*(1-y^2)
 * ref: tanh_activation.cu:13-21, tanh_activation_grad.cu:11-20; tanh.cpp:136-219 */
int cnhip_tanh_forward(const float* x, float* y, int64_t n, cnhip_stream_t stream);
int cnhip_tanh_backward(const float* y, const float* dy, float* dx, int64_t n,
                        cnhip_stream_t stream);

/* ---- losses ------------------------------------------------------------
 * reduction: 0 "mean", 1 "sum".  loss points to ONE device float.      */
#define CNHIP_REDUCE_MEAN 0
#define CNHIP_REDUCE_SUM  1
/* BinaryCrossEntropy on n = rows*cols values; p clipped to [1e-7, 1-1e-7].
 * grad = (p-t)/(p(1-p)) [/n for mean]
 * ref: BinaryCrossEntropy::forward/backward binary_cross_entropy.cpp:143-225 */
int cnhip_bce_forward(const float* pred, const float* target, float* loss,
                      int64_t n, int reduction, cnhip_stream_t stream);
int cnhip_bce_backward(const float* pred, const float* target, float* grad,
                       int64_t n, int reduction, cnhip_stream_t stream);
/* A Sigmoid output layer followed by BinaryCrossEntropy, forward and backward
 * in one launch: p = sigmoid(z), loss = BCE(p, target) (loss_reduction),
 * dz = BCE'(p, target) (grad_reduction) * p (1 - p).  Bit-identical to
 * cnhip_sigmoid_forward + cnhip_bce_forward + cnhip_bce_backward +
 * cnhip_sigmoid_backward (one block: meant for small outputs).
 * ref: sigmoid.cpp:97-231, binary_cross_entropy.cpp:143-225 */
int cnhip_sigmoid_bce_head(const float* z, const float* target, float* p, float* loss, float* dz, int64_t n,
                           int loss_reduction, int grad_reduction, cnhip_stream_t stream);
/* MSE: loss = sum (p-t)^2 [/n]; grad = 2(p-t) [/n]
 * ref: MSE::forward/backward src/CppNet/losses/mse.cpp:102-161 */
int cnhip_mse_forward(const float* pred, const float* target, float* loss,
                      int64_t n, int reduction, cnhip_stream_t stream);
int cnhip_mse_backward(const float* pred, const float* target, float* grad,
                       int64_t n, int reduction, cnhip_stream_t stream);
/* MSE forward and backward in one launch: loss (loss_reduction) and grad
 * (grad_reduction) bit-identical to cnhip_mse_forward + cnhip_mse_backward
 * (one block: meant for small outputs).
 * ref: MSE::forward/backward src/CppNet/losses/mse.cpp:102-161 */
int cnhip_mse_head(const float* pred, const float* target, float* loss, float* grad, int64_t n,
                   int loss_reduction, int grad_reduction, cnhip_stream_t stream);
/* SoftmaxCrossEntropy over ColMajor logits/targets [batch, classes].
 * forward writes the row softmax into softmax_out (the reference's
 * softmax_cache_) and the loss; backward: grad = (softmax - t) [/batch].
 * ref: SoftmaxCrossEntropy::forward/backward softmax_cross_entropy.cpp:118-195 */
int cnhip_softmax_ce_forward(const float* logits, const float* targets,
                             float* softmax_out, float* loss, int64_t batch,
                             int64_t classes, int reduction, cnhip_stream_t stream);
int cnhip_softmax_ce_backward(const float* softmax, const float* targets,
                              float* grad, int64_t batch, int64_t classes,
                              int reduction, cnhip_stream_t stream);
/* SoftmaxCrossEntropy forward and backward together: softmax_out, loss and
 * grad as cnhip_softmax_ce_forward + cnhip_softmax_ce_backward produce them,
 * bit for bit; one launch when batch <= 256, else those two calls. */
int cnhip_softmax_ce_head(const float* logits, const float* targets, float* softmax_out, float* loss,
                          float* grad, int64_t batch, int64_t classes, int reduction, cnhip_stream_t stream);

/* ---- optimizer ---------------------------------------------------------
 * Adam, one tensor: m = b1 m + (1-b1) g ; v = b2 v + (1-b2) g^2 ;
 * W -= lr * (m/bc1) / (sqrt(v/bc2) + eps), bc1/bc2 = 1 - beta^t computed by
 * the caller in float (adam.cpp:121-122).
 * ref: adam_step.cu:10-25; Adam::update src/CppNet/optimizers/adam.cpp:98-133 */
int cnhip_adam_step(float* W, const float* g, float* m, float* v, int64_t n,
                    float lr, float beta1, float beta2, float eps,
                    float bc1, float bc2, cnhip_stream_t stream);
/* The same update over several tensors in ONE launch; tensor i is
 * (W[i], g[i], m[i], v[i], n[i]) with its own bias corrections bc1[i],
 * bc2[i] (the per-key t of the reference).  Host arrays of length count
 * (count <= 64).  ref: as cnhip_adam_step, applied per Layer::step call. */
int cnhip_adam_step_multi(int count, float* const* W, const float* const* g,
                          float* const* m, float* const* v, const int64_t* n,
                          const float* bc1, const float* bc2, float lr,
                          float beta1, float beta2, float eps,
                          cnhip_stream_t stream);
/* One whole training step of Linear(I, H) -> ReLU -> Linear(H, 1) ->
 * Sigmoid with BinaryCrossEntropy and Adam (the reference's quick-start
 * binary classifier, README.md:102-125) in two launches: forward, loss,
 * backward and per-block partial gradient sums (a block per 16 samples),
 * then the gradients (partials added in block order) stored into gW1, gb1,
 * gW2, gb2 (overwritten: the step's own gradients), the loss into *loss
 * (loss_reduction), and Adam applied to W1, b1, W2, b2 in place with moments
 * m[k], v[k] and bias corrections bc1[k], bc2[k] (k = W1, b1, W2, b2; the
 * caller's per-key t).  X [B, I] and Y [B, 1] ColMajor, W1 [I, H] ColMajor.
 * B % 16 == 0, 1 <= I, H <= 64.  Per element the layer-by-layer path's
 * arithmetic; the batch sums in an order of their own.  The Adam update is
 * withheld like cnhip_adam_step_multi's after a faulted recurrence.
 * ref: Linear (linear.cpp:146-358), ReLU (relu.cpp:97-160), Sigmoid
 * (sigmoid.cpp:97-231), BinaryCrossEntropy (binary_cross_entropy.cpp:143-225),
 * Adam::update (adam.cpp:98-133) */
int cnhip_mlp2_bce_adam_step(const float* X, const float* Y, int64_t B, int64_t I, int64_t H,
                             float* W1, float* b1, float* W2, float* b2,
                             float* gW1, float* gb1, float* gW2, float* gb2,
                             float* const* m, float* const* v, const float* bc1, const float* bc2,
                             float lr, float beta1, float beta2, float eps,
                             int loss_reduction, int grad_reduction, float* loss,
                             cnhip_stream_t stream);
/* SGD, Momentum, Adagrad, RMSProp over up to 64 tensors in ONE launch;
 * tensor i is (W[i], g[i], state[i], n[i]), state[i] the per-key velocity,
 * squared-gradient accumulator or mean square (ignored for SGD, may be NULL).
 * hyper is mu (Momentum) or rho (RMSProp); eps is used by Adagrad, RMSProp.
 *   SGD      W -= lr g                                  (sgd.cpp:54-68)
 *   Momentum v = mu v - lr g ; W += v                   (momentum.cpp:81-104)
 *   Adagrad  a += g g ; W -= lr g / (sqrt(a) + eps)     (adagrad.cpp:83-106)
 *   RMSProp  s = rho s + (1 - rho) g g ;
 *            W -= lr g / (sqrt(s) + eps)                (mrs_prop.cpp:83-106)
 * Each evaluated with one rounding per operation, as the reference's host
 * loops (bit-identical for identical inputs).  ref: also sgd_step.cu,
 * momentum_step.cu, adagrad_step.cu, rmsprop_step.cu. */
#define CNHIP_OPT_SGD      0
#define CNHIP_OPT_MOMENTUM 1
#define CNHIP_OPT_ADAGRAD  2
#define CNHIP_OPT_RMSPROP  3
int cnhip_optimizer_step_multi(int kind, int count, float* const* W, const float* const* g,
                               float* const* state, const int64_t* n, float lr, float hyper,
                               float eps, cnhip_stream_t stream);

/* ---- the reference's other device ops ----------------------------------
 * LeakyReLU: y = x > 0 ? x : alpha x ; dx = x > 0 ? dy : alpha dy (the
 * backward reads the INPUT).  ref: LeakyReLU::forward/backward
 * src/CppNet/activations/leacky_relu.cpp:93-229, leaky_relu.cu */
int cnhip_leaky_relu_forward(const float* x, float* y, int64_t n, float alpha,
                             cnhip_stream_t stream);
int cnhip_leaky_relu_backward(const float* x, const float* dy, float* dx, int64_t n,
                              float alpha, cnhip_stream_t stream);
/* Softmax over the LAST dimension of a ColMajor tensor: rows = size / len,
 * element (r, j) at r + rows*j (2-D [B, F]: rows = B; 4-D: rows = d0 d1 d2).
 * backward: dx = y (dy - sum_j dy y).  ref: Softmax::forward/backward
 * src/CppNet/activations/softmax.cpp:105-323 (its gpu branch launches
 * softmax_forward/backward_kernel) */
int cnhip_softmax_forward(const float* x, float* y, int64_t rows, int64_t len,
                          cnhip_stream_t stream);
int cnhip_softmax_backward(const float* y, const float* dy, float* dx, int64_t rows,
                           int64_t len, cnhip_stream_t stream);
/* CategoricalCrossEntropy on ColMajor [B, C] with float (one-hot or soft)
 * targets.  targets_used receives t (1 - ls) + ls / C (a copy of t when
 * label_smoothing == 0); probs receives the softmax of the logits
 * (from_logits) or a copy of the predictions; *loss = sum -t log(clip(p,
 * 1e-15, 1 - 1e-15)), / B for mean.  backward: g = probs - t (from_logits)
 * or -t / clip(p), / B for mean.  The row losses are summed in a fixed
 * order.  ref: CategoricalCrossEntropy::forward/backward
 * src/CppNet/losses/categorical_cross_entropy.cpp:167-380, categorical_ce.cu */
int cnhip_cce_forward(const float* pred, const float* targets, float* probs,
                      float* targets_used, float* loss, int64_t B, int64_t C, int from_logits,
                      float label_smoothing, int reduction, cnhip_stream_t stream);
int cnhip_cce_backward(const float* probs, const float* targets_used, float* grad, int64_t B,
                       int64_t C, int from_logits, int reduction, cnhip_stream_t stream);
/* MAE: mean |p - t|, grad sign(p - t) / n.  Huber(delta): 0.5 d^2 where
 * |d| <= delta, else delta (|d| - delta/2); grad d or delta sign(d), / n for
 * mean.  ref: src/CppNet/losses/mae.cpp:102-160, huber.cpp:104-178 */
int cnhip_mae_forward(const float* p, const float* t, float* loss, int64_t n, int reduction,
                      cnhip_stream_t stream);
int cnhip_mae_backward(const float* p, const float* t, float* grad, int64_t n, int reduction,
                       cnhip_stream_t stream);
int cnhip_huber_forward(const float* p, const float* t, float* loss, int64_t n, float delta,
                        int reduction, cnhip_stream_t stream);
int cnhip_huber_backward(const float* p, const float* t, float* grad, int64_t n, float delta,
                         int reduction, cnhip_stream_t stream);
/* Dropout(p): y = x * mask * 1/(1 - p), mask[i] = 1 with probability 1 - p
 * from a counter-based generator of (seed, offset + i) (the reference draws
 * it from a time-seeded host mt19937, dropout.cpp:19-21); mask is one byte
 * per element, kept for the backward dx = dy * mask * 1/(1 - p).
 * ref: Dropout::forward/backward src/CppNet/layers/dropout.cpp:140-270, dropout.cu */
int cnhip_dropout_forward(const float* x, float* y, uint8_t* mask, int64_t n, float p,
                          uint64_t seed, uint64_t offset, cnhip_stream_t stream);
int cnhip_dropout_backward(const float* dy, const uint8_t* mask, float* dx, int64_t n, float p,
                           cnhip_stream_t stream);
/* Global pools over [N, C, H, W] -> [N, C].  Average: sum over h then w in
 * order, times 1/(H W); backward spreads dY/(H W).  Max: strict > scan (h
 * outer, w inner) from -inf, argmax as int32 (h, w) tensors [N, C]; backward
 * writes dY at the argmax and 0 elsewhere.  ref: GlobalAvgPool2D /
 * GlobalMaxPool2D src/CppNet/layers/global_pool.cpp:111-395,
 * global_avg_pool2d.cu, global_max_pool2d.cu */
int cnhip_global_avgpool_forward(const float* X, float* Y, int64_t N, int64_t C, int64_t H,
                                 int64_t W, cnhip_stream_t stream);
int cnhip_global_avgpool_backward(const float* dY, float* dX, int64_t N, int64_t C, int64_t H,
                                  int64_t W, cnhip_stream_t stream);
int cnhip_global_maxpool_forward(const float* X, float* Y, int32_t* argmax_h, int32_t* argmax_w,
                                 int64_t N, int64_t C, int64_t H, int64_t W,
                                 cnhip_stream_t stream);
int cnhip_global_maxpool_backward(const float* dY, const int32_t* argmax_h,
                                  const int32_t* argmax_w, float* dX, int64_t N, int64_t C,
                                  int64_t H, int64_t W, cnhip_stream_t stream);
/* Elman RNN over X [B, S, I] -> Y [B, S, H]: h_0 = 0,
 * h_t = tanh(x_t W_ih + h_{t-1} W_hh + b); the full sequence is returned.
 * backward OVERWRITES gW_ih, gW_hh, gb and writes dX (may be NULL) from
 * dY [B, S, H] and the forward's Y.  ref: RNN::forward/backward
 * src/CppNet/layers/rnn.cpp:48-171, rnn_cell.cu */
int cnhip_rnn_forward(const float* X, const float* W_ih, const float* W_hh, const float* b,
                      float* Y, int64_t B, int64_t S, int64_t I, int64_t H,
                      cnhip_stream_t stream);
int cnhip_rnn_backward(const float* X, const float* W_ih, const float* W_hh, const float* Y,
                       const float* dY, float* gW_ih, float* gW_hh, float* gb, float* dX,
                       int64_t B, int64_t S, int64_t I, int64_t H, cnhip_stream_t stream);

/* ---- DataLoader batch assembly (ref: dataloader.cpp:68-88) ----
 * src: the dataset sample-major (sample n's F values at src + n*F), N
 * samples; idx: B int32 sample indices (one outside [0, N) yields zeros);
 * dst: the batch ColMajor [B, F], dst[b + B*f] = src[idx[b]*F + f]. */
int cnhip_gather_rows(const float* src, const int32_t* idx, float* dst, int64_t N, int64_t F, int64_t B,
                      cnhip_stream_t stream);
/* Features and labels of one batch in one launch: xs [N samples x F] and
 * ys [N x L] sample-major -> x [B, F], y [B, L] ColMajor. */
int cnhip_gather_batch(const float* xs, const float* ys, const int32_t* idx, float* x, float* y, int64_t N,
                       int64_t F, int64_t L, int64_t B, cnhip_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* CNHIP_H */
