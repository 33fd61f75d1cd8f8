/*
 * cppnet_train.h — C ABI of the C++17 training harness (libcppnet.so).
 *
 * A session owns one model built from the CppNet-compatible layer classes
 * (device "gpu"), its loss, an Adam optimizer, a dedicated HIP stream and the
 * current batch, all resident in HBM.  cnt_step() runs exactly the
 * reference harness's train step (benchmarks/mlp_benchmark.cpp:166-175):
 *   model.zero_grad(); out = model.forward(X); loss = loss_fn.forward(out, Y);
 *   g = loss_fn.backward(out, Y); model.backward(g); model.update(adam, lr)
 * Parameters are indexed in layer order, weight before bias.  Host buffers
 * are ColMajor float32 (Eigen's order).  Functions return 0 on success and
 * a cnhip status code otherwise; cnt_last_error() has the message.
 */
#ifndef CPPNET_TRAIN_H
#define CPPNET_TRAIN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct cnt_session cnt_session;

#define CNT_ACT_NONE    0
#define CNT_ACT_RELU    1
#define CNT_ACT_SIGMOID 2
#define CNT_ACT_TANH    3
#define CNT_ACT_LEAKY_RELU 4 /* alpha 0.01 (leacky_relu.hpp default) */
#define CNT_ACT_SOFTMAX    5 /* over the features of each row */

#define CNT_LOSS_BCE        0
#define CNT_LOSS_SOFTMAX_CE 1
#define CNT_LOSS_MSE        2
#define CNT_LOSS_CCE        3 /* CategoricalCrossEntropy("mean", from_logits) */
#define CNT_LOSS_MAE        4 /* MAE("mean") */
#define CNT_LOSS_HUBER      5 /* Huber(delta 1, "mean") */

/* optimizers of cnt_set_optimizer */
#define CNT_OPT_ADAM     0
#define CNT_OPT_SGD      1
#define CNT_OPT_MOMENTUM 2 /* hyper = mu */
#define CNT_OPT_ADAGRAD  3 /* eps */
#define CNT_OPT_RMSPROP  4 /* hyper = rho, eps */

const char* cnt_last_error(void);

/* MLP: n_linear Linear layers with sizes[0] -> sizes[1] -> ... -> sizes[n_linear]
 * (xavier init, bias), hidden_act after every layer but the last, out_act after
 * the last, the given loss ("mean"), Adam(beta1, beta2, eps) at rate lr, batch
 * rows per step.  Configs 1 and 2 of the benchmark are instances of it.
 * ref: benchmarks/mlp_benchmark.cpp:85-192; README.md:112-137 */
int cnt_mlp_create(cnt_session** out, int n_linear, const int64_t* sizes, int hidden_act,
                   int out_act, int loss, int64_t batch, float lr, float beta1, float beta2,
                   float eps, uint64_t seed);
/* The same with Dropout(dropout) after every hidden activation (dropout in
 * [0, 1); 0 adds none).  Checkpoints save and restore the Dropout layers'
 * mask-generator positions.  ref: src/CppNet/layers/dropout.cpp:15-270 */
int cnt_mlp_create_ex(cnt_session** out, int n_linear, const int64_t* sizes, int hidden_act,
                      int out_act, int loss, int64_t batch, float lr, float beta1, float beta2,
                      float eps, uint64_t seed, float dropout);
/* CNN: n_conv blocks of Conv2D(in, out, kernel, stride, padding; bias) -> ReLU
 * -> MaxPool2D(pool), conv_spec holding 5 values per block; then Flatten ->
 * Linear(C*H*W -> classes) -> SoftmaxCrossEntropy("mean"), Adam.  input_shape
 * is [N, C, H, W].  Config 3 of the benchmark is an instance of it.
 * ref: benchmarks/cnn_benckmark.cpp:94-291 (caller pattern) */
int cnt_cnn_create(cnt_session** out, int n_conv, const int64_t* conv_spec, int pool,
                   const int64_t* input_shape, int64_t classes, float lr, float beta1,
                   float beta2, float eps, uint64_t seed);
/* Sequence regressor: LSTM (cell 0), GRU (cell 1) or Elman RNN (cell 2) over X [batch, seq_len,
 * input_size] -> last hidden state -> Linear(hidden -> out_features) ->
 * MSE("mean"), Adam.  Parameters: W_ih, W_hh, b of the cell, then W, b of the
 * Linear.  Config 4 of the benchmark is the LSTM instance.
 * ref: benchmarks/sequence_benckmark.cpp:64-192 (caller pattern) */
int cnt_rnn_create(cnt_session** out, int cell, int64_t batch, int64_t seq_len,
                   int64_t input_size, int64_t hidden_size, int64_t out_features, float lr,
                   float beta1, float beta2, float eps, uint64_t seed);
/* Residual MLP, the reference's residual benchmark network
 * (benchmarks/residual_benckmark.cpp:104-152): Linear(in_features -> width,
 * "he") -> ReLU -> depth x [Residual({Linear(w -> width, "he"), Linear(width
 * -> w', "he")}, w, w') -> ReLU] -> Linear(w_last -> classes, "xavier") ->
 * SoftmaxCrossEntropy("mean"), Adam.  w = width for every block; w' = width
 * except for the last block, whose w' = last_width (a bias-free projection
 * shortcut when last_width != width, residual.cpp:31-36).  Parameters:
 * proj W, b; per block fc_a W, b, fc_b W, b [, projection W]; head W, b.
 * ref: Residual::forward/backward/step src/CppNet/layers/residual.cpp:23-159 */
int cnt_resnet_create(cnt_session** out, int64_t in_features, int64_t width, int depth, int64_t last_width,
                      int64_t classes, int64_t batch, float lr, float beta1, float beta2, float eps,
                      uint64_t seed);
/* Transformer encoder classifier (config 5): Embedding(vocab, D) -> n_blocks x
 * [r = MultiHeadAttention(D, heads)(x, x, x) + x; h = BatchNorm(D) on the
 * [B*S, D] view; y = Linear(ffn -> D)(GELU(Linear(D -> ffn)(h))) + h] ->
 * MeanPool1D -> Linear(D -> classes) -> SoftmaxCrossEntropy("mean"), Adam.
 * Inputs are int32 token ids [batch, seq_len] (cnt_set_batch_tokens).
 * Parameters: the embedding table (ColMajor [vocab, D] on the host side),
 * then per block W_q, W_k, W_v, W_o, gamma, beta, W1, b1, W2, b2, then the
 * classifier W, b.
 * ref: the harness composition of benchmarks/transformer_benckmark.cpp:95-175
 * with the layers of src/CppNet/layers/{embedding,attention,batch_norm,
 * mean_pool1d}.cpp */
int cnt_transformer_create(cnt_session** out, int64_t batch, int64_t seq_len, int64_t vocab,
                           int64_t embed_dim, int64_t heads, int n_blocks, int64_t ffn_dim,
                           int64_t classes, float lr, float beta1, float beta2, float eps,
                           uint64_t seed);
int cnt_destroy(cnt_session* s);
/* Replaces the session's optimizer (Adam from the create call) before its
 * first update: kind CNT_OPT_*; hyper is Momentum's mu or RMSProp's rho
 * (ignored otherwise), eps Adagrad's / RMSProp's epsilon; CNT_OPT_ADAM takes
 * beta1 = hyper and eps with beta2 0.999.  State starts at zero.  Refused
 * once the session has updated (the reference's optimizers keep per-parameter
 * state that a swap would drop).
 * ref: src/CppNet/optimizers/{sgd,momentum,adagrad,mrs_prop,adam}.cpp */
int cnt_set_optimizer(cnt_session* s, int kind, float hyper, float eps);

int cnt_num_params(cnt_session* s, int* count);
int cnt_param_size(cnt_session* s, int index, int64_t* n);
int cnt_set_param(cnt_session* s, int index, const float* host);
int cnt_get_param(cnt_session* s, int index, float* host);
int cnt_get_grad(cnt_session* s, int index, float* host);
/* Host copy of the optimizer's state tensor k of parameter `index` (Adam: 0
 * m, 1 v; Momentum, Adagrad, RMSProp: 0 their one tensor; in the layout of
 * cnt_get_param) and its step count *t (Adam's per-key t; 0 and zeros
 * before the parameter's first update).  No counterpart in the reference,
 * whose optimizer state is private (adam.hpp:40-53). */
int cnt_get_opt_state(cnt_session* s, int index, int k, float* host, int* t);

/* Uploads one batch (X: the model's input shape, Y: [batch, outputs]) that
 * every later cnt_step() trains on, until the next call. */
int cnt_set_batch(cnt_session* s, const float* x_host, const float* y_host);
/* Transformer sessions: int32 token ids [batch, seq_len] and one-hot Y. */
int cnt_set_batch_tokens(cnt_session* s, const int32_t* ids_host, const float* y_host);
/* Same from device memory already in HBM (copied on the session stream). */
int cnt_set_batch_device(cnt_session* s, const float* x_dev, const float* y_dev);

/* One train step.  loss_out == NULL keeps the step fully asynchronous;
 * otherwise the stream is synchronised and the step's loss written. */
int cnt_step(cnt_session* s, float* loss_out);
/* The two halves of cnt_step: zero_grad + forward + loss + backward (grads
 * are readable afterwards), then the optimizer update.  Conv2D clears its
 * gradients inside step() (conv2d.cpp:211-212), so read grads in between. */
int cnt_forward_backward(cnt_session* s, float* loss_out);
int cnt_update(cnt_session* s);
/* Fused steps (on by default): cnt_step on a session of Linear(I, H) ->
 * ReLU -> Linear(H, 1) -> Sigmoid with BinaryCrossEntropy and Adam (the
 * reference's MLP benchmark model; I, H <= 64, batch % 16 == 0) runs each
 * step as two launches (cnhip_mlp2_bce_adam_step) instead of seven
 * layer-by-layer ones (a capture after fused steps first runs one
 * layer-by-layer forward + backward, without an update, to size its
 * buffers).  Per element the same arithmetic; the sums
 * over the batch are ordered per 16-sample block, so its gradients differ
 * from the layer-by-layer step's in the last bits.  enable = 0 keeps every
 * step layer by layer (for bitwise comparisons with a captured graph, which
 * always replays the layer-by-layer kernels).  No counterpart in the
 * reference. */
int cnt_set_fused_step(cnt_session* s, int enable);
/* Whole-step graph.  cnt_capture_step records the session's zero_grad +
 * forward + loss + backward into a HIP graph (include/cnhip.h, graphs);
 * from then on cnt_step replays it with one graph launch and then runs the
 * Adam update eagerly (its bias corrections 1 - beta^t change every step and
 * are computed on the host exactly as the eager path does), so a replayed
 * step computes what an eager layer-by-layer step computes, bit for bit.  Needs one eager
 * step (cnt_step or cnt_forward_backward) at the session's shapes first.
 * The graph reads the batch buffers in place, so cnt_set_batch* between
 * replays trains on the new batch.  cnt_forward_backward runs eagerly and
 * drops the graph (the layers' cached activations then belong to that
 * pass); so does cnt_release_graph.  No counterpart in the reference. */
int cnt_capture_step(cnt_session* s);
int cnt_release_graph(cnt_session* s);
int cnt_has_graph(cnt_session* s); /* 1 while a captured graph is live */
int cnt_synchronize(cnt_session* s);

/* Model files.  cnt_save_model / cnt_load_model: the reference's "CNET"
 * format exactly (Utils::save_model / load_model,
 * ref: src/CppNet/utils/serialization.cpp:143-256): magic 0x434E4554, the
 * layer count, then per trainable layer a type id (Linear 1: W [in, out],
 * b; BatchNorm 2: gamma, beta, running mean, running var; Embedding 3: the
 * [vocab, dim] table; other 0, no data) with int32-ndims/dims + float32
 * ColMajor records.  cnt_save_checkpoint / cnt_load_checkpoint write the
 * same records followed by an extension the reference's reader ignores:
 * every parameter's values and the optimizer's per-parameter state and step
 * counts, so a loaded session continues exactly as the saved one would have
 * (no counterpart in the reference, whose files hold weights only). */
int cnt_save_model(cnt_session* s, const char* path);
int cnt_load_model(cnt_session* s, const char* path);
int cnt_save_checkpoint(cnt_session* s, const char* path);
int cnt_load_checkpoint(cnt_session* s, const char* path);

/* .npy v1.0 float32 files (Utils::save_npy / load_npy_*,
 * ref: src/CppNet/utils/tensor_io.cpp:29-170).  Data is ColMajor; the writer
 * says 'fortran_order': True so that numpy.load returns the logical array
 * (the reference writes the same bytes under False).  The reader follows the
 * file's flag, reordering C-order data into ColMajor; raw_colmajor = 1 takes
 * the bytes as ColMajor whatever the flag (files the reference wrote).
 * cnt_npy_load: on entry *ndims is the capacity of dims and capacity that of
 * out (floats); on return they hold the rank, shape and data.  Host-only. */
/* DataLoader (Utils::DataLoader, ref: include/CppNet/utils/dataloader.hpp:46-109,
 * src/CppNet/utils/dataloader.cpp:12-120): features [N, F] and labels [N, L]
 * (host, ColMajor; copied), batch size, shuffle, drop_last; the shuffle is
 * std::shuffle with a std::mt19937 seeded by `seed`.  cnt_loader_host_batch
 * is the reference's batch k on the host (*bs = its size).  After
 * cnt_loader_to_device (CNT_STAGE_RESIDENT: the dataset in HBM, batches
 * gathered on the GPU; CNT_STAGE_STREAM: page-locked double-buffered uploads
 * on a copy stream, overlapping the caller's work), cnt_loader_next writes the
 * epoch's next batch ColMajor into device buffers on `stream`, and
 * cnt_loader_next_batch into a session's batch (same as cnt_set_batch_device;
 * MLP, CNN and sequence sessions: the session's batch size must match);
 * *bs = 0 at the end of the epoch.  cnt_loader_reset reshuffles and
 * restarts the epoch. */
typedef struct cnt_loader cnt_loader;
#define CNT_STAGE_RESIDENT 1
#define CNT_STAGE_STREAM   2
int cnt_loader_create(cnt_loader** out, const float* features, const float* labels, int64_t n,
                      int64_t f, int64_t l, int64_t batch, int shuffle, int drop_last, uint64_t seed);
int cnt_loader_destroy(cnt_loader* ld);
int cnt_loader_num_batches(cnt_loader* ld, int64_t* count);
int cnt_loader_indices(cnt_loader* ld, int32_t* out); /* the epoch's order, n entries */
int cnt_loader_reset(cnt_loader* ld);
int cnt_loader_host_batch(cnt_loader* ld, int64_t k, float* x, float* y, int64_t* bs);
int cnt_loader_to_device(cnt_loader* ld, int mode);
int cnt_loader_next(cnt_loader* ld, float* x_dev, float* y_dev, int64_t* bs, void* stream);
int cnt_loader_next_batch(cnt_loader* ld, cnt_session* s, int64_t* bs);

int cnt_npy_save(const char* path, const float* colmajor, int ndims, const int64_t* dims);
int cnt_npy_load(const char* path, float* out, int64_t capacity, int* ndims, int64_t* dims,
                 int raw_colmajor);
/* The hipStream_t the session's kernels run on. */
void* cnt_stream(cnt_session* s);

#ifdef __cplusplus
}
#endif
#endif
