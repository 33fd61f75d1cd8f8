"""Thin torch-tensor front end to the C ABI (include/cnhip.h).

Tensors are device tensors holding Eigen ColMajor data: a CppNet
``[rows, cols]`` matrix is a flat (or any contiguous) float32 tensor of
rows*cols values with the row index fastest.  torch is used only for device
memory and the current stream; every computation is a HIP kernel of
libcnhip.so.  Entry points raise CnhipError (with cnhip_last_error()) on a
non-zero status and refuse host tensors.
"""
from __future__ import annotations

import torch

from . import _capi

MEAN, SUM = 0, 1
_REDUCTIONS = {"mean": MEAN, "sum": SUM}


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _p(t: torch.Tensor | None, name: str = "tensor") -> int | None:
    if t is None:
        return None
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"{name}: expected a device tensor (the HIP path has no host fallback)")
    if t.dtype not in (torch.float32, torch.int32, torch.uint8):
        raise TypeError(f"{name}: expected float32/int32/uint8, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: expected a contiguous tensor")
    return t.data_ptr()


def _red(reduction: str | int) -> int:
    if isinstance(reduction, int):
        return reduction
    if reduction not in _REDUCTIONS:
        raise ValueError(f'reduction must be "mean" or "sum", got {reduction!r}')
    return _REDUCTIONS[reduction]


def gemm(trans_a: bool, trans_b: bool, M: int, N: int, K: int, A, lda: int, B, ldb: int, C,
         ldc: int, alpha: float = 1.0, beta: float = 0.0, bias=None, relu: bool = False) -> None:
    _capi.call("cnhip_gemm_f32", int(trans_a), int(trans_b), M, N, K, alpha, _p(A, "A"), lda,
               _p(B, "B"), ldb, beta, _p(C, "C"), ldc, _p(bias, "bias"), 1 if relu else 0,
               _stream())


def gemm_batched(trans_a: bool, trans_b: bool, M: int, N: int, K: int, A, lda: int, sa: int, B,
                 ldb: int, sb: int, C, ldc: int, sc: int, batch: int, alpha: float = 1.0,
                 beta: float = 0.0) -> None:
    _capi.call("cnhip_gemm_f32_batched", int(trans_a), int(trans_b), M, N, K, alpha, _p(A, "A"),
               lda, sa, _p(B, "B"), ldb, sb, beta, _p(C, "C"), ldc, sc, batch, _stream())


def linear_forward(X, W, b, Y, batch: int, in_features: int, out_features: int) -> None:
    _capi.call("cnhip_linear_forward", _p(X, "X"), _p(W, "W"), _p(b, "b"), _p(Y, "Y"), batch,
               in_features, out_features, _stream())


def linear_backward(X, W, dY, grad_W, grad_b, dX, batch: int, in_features: int,
                    out_features: int, trainable: bool = True, accumulate: bool = True) -> None:
    _capi.call("cnhip_linear_backward", _p(X, "X"), _p(W, "W"), _p(dY, "dY"),
               _p(grad_W, "grad_W"), _p(grad_b, "grad_b"), _p(dX, "dX"), batch, in_features,
               out_features, int(trainable), int(accumulate), _stream())


ACT = {"none": 0, "relu": 1, "gelu": 2, "residual": 3}


def linear_forward_act(X, W, b, Y, Z, batch: int, in_features: int, out_features: int,
                       act: str) -> None:
    _capi.call("cnhip_linear_forward_act", _p(X), _p(W), _p(b), _p(Y), _p(Z), batch, in_features,
               out_features, ACT[act], _stream())


def linear_backward_act(X, W, dY, grad_W, grad_b, dX, act_aux, batch: int, in_features: int,
                        out_features: int, act: str, trainable: bool = True,
                        accumulate: bool = False) -> None:
    _capi.call("cnhip_linear_backward_act", _p(X), _p(W), _p(dY), _p(grad_W), _p(grad_b), _p(dX),
               _p(act_aux), batch, in_features, out_features, int(trainable), int(accumulate),
               ACT[act], _stream())


def linear_backward_act_noalloc(X, W, dY, grad_W, grad_b, dX, act_aux, batch: int, in_features: int,
                                out_features: int, act: str, trainable: bool = True,
                                accumulate: bool = False) -> None:
    """linear_backward_act with its workspace in the library's fixed device
    array (no device allocation); shapes that need more are refused."""
    _capi.call("cnhip_linear_backward_act_noalloc", _p(X), _p(W), _p(dY), _p(grad_W), _p(grad_b), _p(dX),
               _p(act_aux), batch, in_features, out_features, int(trainable), int(accumulate),
               ACT[act], _stream())


def column_sum(x, out, rows: int, cols: int, accumulate: bool = False) -> None:
    _capi.call("cnhip_column_sum", _p(x), _p(out), rows, cols, int(accumulate), _stream())


def conv2d_forward(X, W, b, Y, N, C, H, Wd, OC, KS, S=1, P=0) -> None:
    _capi.call("cnhip_conv2d_forward", _p(X, "X"), _p(W, "W"), _p(b, "b"), _p(Y, "Y"), N, C, H, Wd,
               OC, KS, S, P, _stream())


def conv2d_forward_relu(X, W, b, Y, N, C, H, Wd, OC, KS, S=1, P=0) -> None:
    """Conv2D forward with the following ReLU in its epilogue: Y = max(0, conv + b)."""
    _capi.call("cnhip_conv2d_forward_relu", _p(X, "X"), _p(W, "W"), _p(b, "b"), _p(Y, "Y"), N, C,
               H, Wd, OC, KS, S, P, _stream())


def conv2d_forward_relu_maxpool(X, W, b, Yp, idx, N, C, H, Wd, OC, KS, S=1, P=0, pool=2, pool_stride=-1) -> None:
    """Conv2D forward, ReLU and MaxPool2D in one call: Yp the pooled output, idx its argmax."""
    _capi.call("cnhip_conv2d_forward_relu_maxpool", _p(X, "X"), _p(W, "W"), _p(b, "b"), _p(Yp, "Yp"),
               _p(idx, "idx"), N, C, H, Wd, OC, KS, S, P, pool, pool_stride, _stream())


def conv2d_backward(X, W, dY, grad_W, grad_b, dX, N, C, H, Wd, OC, KS, S=1, P=0) -> None:
    _capi.call("cnhip_conv2d_backward", _p(X, "X"), _p(W, "W"), _p(dY, "dY"), _p(grad_W, "gW"),
               _p(grad_b, "gb"), _p(dX, "dX"), N, C, H, Wd, OC, KS, S, P, _stream())


def conv2d_backward_maxpool_relu(X, dP, idx, Pout, grad_W, grad_b, N, C, H, Wd, OC, KS, S=1, P=0, pool=2,
                                 pool_stride=-1) -> None:
    """Weight and bias gradients of Conv2D -> ReLU -> MaxPool2D from the pooled gradient."""
    _capi.call("cnhip_conv2d_backward_maxpool_relu", _p(X, "X"), _p(dP, "dP"), _p(idx, "idx"), _p(Pout, "Pout"),
               _p(grad_W, "gW"), _p(grad_b, "gb"), N, C, H, Wd, OC, KS, S, P, pool, pool_stride, _stream())


def conv2d_backward_maxpool_relu_fits(N, C, H, Wd, OC, KS, S=1, P=0, pool=2, pool_stride=-1) -> bool:
    return bool(_capi.load().cnhip_conv2d_backward_maxpool_relu_fits(N, C, H, Wd, OC, KS, S, P, pool, pool_stride))


def maxpool2d_forward(X, Y, idx, N, C, H, W, pool=2, stride=-1) -> None:
    _capi.call("cnhip_maxpool2d_forward", _p(X, "X"), _p(Y, "Y"), _p(idx, "idx"), N, C, H, W,
               pool, stride, _stream())


def maxpool2d_backward(dY, idx, dX, N, C, H, W, pool=2, stride=-1) -> None:
    _capi.call("cnhip_maxpool2d_backward", _p(dY, "dY"), _p(idx, "idx"), _p(dX, "dX"), N, C, H, W,
               pool, stride, _stream())


def maxpool2d_backward_relu(dY, idx, y, dX, N, C, H, W, pool=2, stride=-1) -> None:
    """MaxPool2D backward times the mask [y > 0] of the ReLU output y feeding the pool."""
    _capi.call("cnhip_maxpool2d_backward_relu", _p(dY, "dY"), _p(idx, "idx"), _p(y, "y"),
               _p(dX, "dX"), N, C, H, W, pool, stride, _stream())


def maxpool2d_backward_relu_pooled(dY, idx, Y, dX, N, C, H, W, pool=2, stride=-1) -> None:
    """MaxPool2D backward times the ReLU mask, taken from the pool's output Y."""
    _capi.call("cnhip_maxpool2d_backward_relu_pooled", _p(dY, "dY"), _p(idx, "idx"), _p(Y, "Y"),
               _p(dX, "dX"), N, C, H, W, pool, stride, _stream())


def linear_backward_maxpool_relu(P, idx, W, dZ, gW, gb, dX, N, C, H, Wd, out_features, pool=2, stride=-1,
                                 accumulate=0) -> None:
    """Backward of Conv2D -> ReLU -> MaxPool2D -> Flatten -> Linear from the
    Linear's output gradient dZ: gW (+)= P^T dZ, gb (+)= column sums of dZ, and
    dX (the ReLU input's gradient) = the pool's routing of (dZ W^T) * [P > 0]."""
    _capi.call("cnhip_linear_backward_maxpool_relu", _p(P, "P"), _p(idx, "idx"), _p(W, "W"), _p(dZ, "dZ"),
               _p(gW, "gW"), _p(gb), _p(dX, "dX"), N, C, H, Wd, out_features, pool,
               stride, accumulate, _stream())


def linear_backward_maxpool_relu_fits(N, C, H, Wd, out_features, pool=2, stride=-1) -> bool:
    return bool(_capi.load().cnhip_linear_backward_maxpool_relu_fits(N, C, H, Wd, out_features, pool, stride))


def lstm_forward(X, W_ih, W_hh, b, Y, gates, c, tanh_c, B, S, I, H) -> None:
    _capi.call("cnhip_lstm_forward", *(_p(t) for t in (X, W_ih, W_hh, b, Y, gates, c, tanh_c)),
               B, S, I, H, _stream())


def lstm_backward(X, W_ih, W_hh, Y, gates, c, tanh_c, dY, gW_ih, gW_hh, gb, dX, B, S, I, H):
    _capi.call("cnhip_lstm_backward", *(_p(t) for t in (X, W_ih, W_hh, Y, gates, c, tanh_c, dY,
                                                        gW_ih, gW_hh, gb, dX)), B, S, I, H,
               _stream())


def lstm_backward_last(X, W_ih, W_hh, Y, gates, c, tanh_c, dY_last, gW_ih, gW_hh, gb, dX, B, S, I, H):
    """lstm_backward for a gradient dY_last [B, H] of the last step's output only."""
    _capi.call("cnhip_lstm_backward_last", *(_p(t) for t in (X, W_ih, W_hh, Y, gates, c, tanh_c, dY_last,
                                                             gW_ih, gW_hh, gb, dX)), B, S, I, H,
               _stream())


def gru_forward(X, W_ih, W_hh, b, Y, gates, rh, B, S, I, H) -> None:
    _capi.call("cnhip_gru_forward", *(_p(t) for t in (X, W_ih, W_hh, b, Y, gates, rh)), B, S, I, H,
               _stream())


def gru_backward(X, W_ih, W_hh, Y, gates, rh, dY, gW_ih, gW_hh, gb, dX, B, S, I, H) -> None:
    _capi.call("cnhip_gru_backward", *(_p(t) for t in (X, W_ih, W_hh, Y, gates, rh, dY, gW_ih,
                                                       gW_hh, gb, dX)), B, S, I, H, _stream())


def seq_select(Y, out, B, S, D, t) -> None:
    _capi.call("cnhip_seq_select", _p(Y), _p(out), B, S, D, t, _stream())


def seq_scatter(inp, Y, B, S, D, t) -> None:
    _capi.call("cnhip_seq_scatter", _p(inp), _p(Y), B, S, D, t, _stream())


def transpose(inp, out, rows: int, cols: int) -> None:
    _capi.call("cnhip_transpose", _p(inp), _p(out), rows, cols, _stream())


def mha_cache_floats(B: int, S: int, D: int) -> int:
    return int(_capi.load().cnhip_mha_cache_floats(B, S, D))


def mha_forward(q, k, v, Wq, Wk, Wv, Wo, out, cache, B, S, D, heads) -> None:
    _capi.call("cnhip_mha_forward", *(_p(t) for t in (q, k, v, Wq, Wk, Wv, Wo, out, cache)),
               B, S, D, heads, _stream())


def mha_backward(q, k, v, Wq, Wk, Wv, Wo, cache, dY, gWq, gWk, gWv, gWo, dX, B, S, D,
                 heads) -> None:
    _capi.call("cnhip_mha_backward", *(_p(t) for t in (q, k, v, Wq, Wk, Wv, Wo, cache, dY, gWq,
                                                       gWk, gWv, gWo, dX)), B, S, D, heads,
               _stream())


# Row order of [B, S, D] sequences: ROWS_REF = row b + B*s of [B*S, D] (the
# reference's), ROWS_BY_SAMPLE = row s + S*b.  rows=ROWS_REF calls the
# reference-layout entry point itself.
ROWS_REF, ROWS_BY_SAMPLE = 0, 1


def mha_forward_residual(q, k, v, Wq, Wk, Wv, Wo, residual, out, cache, B, S, D, heads,
                         rows=ROWS_REF) -> None:
    ptrs = [_p(t) for t in (q, k, v, Wq, Wk, Wv, Wo, residual, out, cache)]
    if rows == ROWS_REF:
        _capi.call("cnhip_mha_forward_residual", *ptrs, B, S, D, heads, _stream())
    else:
        _capi.call("cnhip_mha_forward_rows", *ptrs, B, S, D, heads, rows, _stream())


def mha_backward_residual(q, k, v, Wq, Wk, Wv, Wo, cache, dY, skip_grad, gWq, gWk, gWv, gWo, dX,
                          B, S, D, heads, rows=ROWS_REF) -> None:
    ptrs = [_p(t) for t in (q, k, v, Wq, Wk, Wv, Wo, cache, dY, skip_grad, gWq, gWk, gWv, gWo, dX)]
    if rows == ROWS_REF:
        _capi.call("cnhip_mha_backward_residual", *ptrs, B, S, D, heads, _stream())
    else:
        _capi.call("cnhip_mha_backward_rows", *ptrs, B, S, D, heads, rows, _stream())


def embedding_forward(ids, Wt, out, B, S, V, D, oob=None, rows=ROWS_REF) -> None:
    if rows == ROWS_REF:
        _capi.call("cnhip_embedding_forward", _p(ids), _p(Wt), _p(out), B, S, V, D, _p(oob),
                   _stream())
    else:
        _capi.call("cnhip_embedding_forward_rows", _p(ids), _p(Wt), _p(out), B, S, V, D, _p(oob),
                   rows, _stream())


def embedding_backward(ids, dY, gWt, B, S, V, D, rows=ROWS_REF) -> None:
    if rows == ROWS_REF:
        _capi.call("cnhip_embedding_backward", _p(ids), _p(dY), _p(gWt), B, S, V, D, _stream())
    else:
        _capi.call("cnhip_embedding_backward_rows", _p(ids), _p(dY), _p(gWt), B, S, V, D, rows,
                   _stream())


def batchnorm_forward(x, y, xhat, gamma, beta, rmean, rvar, bmean, bvar, N, F, momentum=0.1,
                      eps=1e-5) -> None:
    _capi.call("cnhip_batchnorm_forward", *(_p(t) for t in (x, y, xhat, gamma, beta, rmean, rvar,
                                                            bmean, bvar)), N, F, momentum, eps,
               _stream())


def batchnorm_backward(dY, x, xhat, gamma, bmean, bvar, ggamma, gbeta, dX, N, F,
                       eps=1e-5) -> None:
    _capi.call("cnhip_batchnorm_backward", *(_p(t) for t in (dY, x, xhat, gamma, bmean, bvar,
                                                             ggamma, gbeta, dX)), N, F, eps,
               _stream())


def gelu_forward(x, y) -> None:
    _capi.call("cnhip_gelu_forward", _p(x), _p(y), x.numel(), _stream())


def gelu_backward(x, dy, dx) -> None:
    _capi.call("cnhip_gelu_backward", _p(x), _p(dy), _p(dx), x.numel(), _stream())


def meanpool1d_forward(x, y, B, S, D, rows=ROWS_REF) -> None:
    if rows == ROWS_REF:
        _capi.call("cnhip_meanpool1d_forward", _p(x), _p(y), B, S, D, _stream())
    else:
        _capi.call("cnhip_meanpool1d_forward_rows", _p(x), _p(y), B, S, D, rows, _stream())


def meanpool1d_backward(dy, dx, B, S, D, rows=ROWS_REF) -> None:
    if rows == ROWS_REF:
        _capi.call("cnhip_meanpool1d_backward", _p(dy), _p(dx), B, S, D, _stream())
    else:
        _capi.call("cnhip_meanpool1d_backward_rows", _p(dy), _p(dx), B, S, D, rows, _stream())


def add(a, b, y) -> None:
    _capi.call("cnhip_add", _p(a), _p(b), _p(y), a.numel(), _stream())


def _unary(name: str, x, y) -> None:
    _capi.call(name, _p(x, "x"), _p(y, "y"), x.numel(), _stream())


def _binary(name: str, y, dy, dx) -> None:
    if not (y.numel() == dy.numel() == dx.numel()):
        raise ValueError(f"{name}: size mismatch")
    _capi.call(name, _p(y, "y"), _p(dy, "dy"), _p(dx, "dx"), y.numel(), _stream())


def relu_forward(x, y): _unary("cnhip_relu_forward", x, y)
def relu_backward(y, dy, dx): _binary("cnhip_relu_backward", y, dy, dx)
def sigmoid_forward(x, y): _unary("cnhip_sigmoid_forward", x, y)
def sigmoid_backward(y, dy, dx): _binary("cnhip_sigmoid_backward", y, dy, dx)
def tanh_forward(x, y): _unary("cnhip_tanh_forward", x, y)
def tanh_backward(y, dy, dx): _binary("cnhip_tanh_backward", y, dy, dx)


def bce_forward(pred, target, loss, reduction="mean") -> None:
    _capi.call("cnhip_bce_forward", _p(pred), _p(target), _p(loss), pred.numel(),
               _red(reduction), _stream())


def bce_backward(pred, target, grad, reduction="mean") -> None:
    _capi.call("cnhip_bce_backward", _p(pred), _p(target), _p(grad), pred.numel(),
               _red(reduction), _stream())


def mse_forward(pred, target, loss, reduction="mean") -> None:
    _capi.call("cnhip_mse_forward", _p(pred), _p(target), _p(loss), pred.numel(),
               _red(reduction), _stream())


def mse_backward(pred, target, grad, reduction="mean") -> None:
    _capi.call("cnhip_mse_backward", _p(pred), _p(target), _p(grad), pred.numel(),
               _red(reduction), _stream())


def mse_head(pred, target, loss, grad, reduction="mean") -> None:
    """mse_forward and mse_backward in one launch (the same bits)."""
    _capi.call("cnhip_mse_head", _p(pred), _p(target), _p(loss), _p(grad), pred.numel(),
               _red(reduction), _red(reduction), _stream())


def softmax_ce_forward(logits, targets, softmax_out, loss, batch: int, classes: int,
                       reduction="mean") -> None:
    _capi.call("cnhip_softmax_ce_forward", _p(logits), _p(targets), _p(softmax_out), _p(loss),
               batch, classes, _red(reduction), _stream())


def softmax_ce_backward(softmax, targets, grad, batch: int, classes: int,
                        reduction="mean") -> None:
    _capi.call("cnhip_softmax_ce_backward", _p(softmax), _p(targets), _p(grad), batch, classes,
               _red(reduction), _stream())


def adam_step(W, g, m, v, lr: float, beta1: float, beta2: float, eps: float, bc1: float,
              bc2: float) -> None:
    _capi.call("cnhip_adam_step", _p(W), _p(g), _p(m), _p(v), W.numel(), lr, beta1, beta2, eps,
               bc1, bc2, _stream())


def adam_step_multi(params: list, lr: float, beta1: float, beta2: float, eps: float) -> None:
    """params: list of (W, g, m, v, bc1, bc2) device-tensor tuples."""
    import ctypes as C
    n = len(params)
    arr = lambda idx: (C.c_void_p * n)(*[_p(p[idx]) for p in params])
    sizes = (C.c_int64 * n)(*[p[0].numel() for p in params])
    bc1 = (C.c_float * n)(*[p[4] for p in params])
    bc2 = (C.c_float * n)(*[p[5] for p in params])
    _capi.call("cnhip_adam_step_multi", n, arr(0), arr(1), arr(2), arr(3), sizes, bc1, bc2, lr,
               beta1, beta2, eps, _stream())


# ---------------------------------------------------------------- the reference's other device ops
OPT = {"sgd": 0, "momentum": 1, "adagrad": 2, "rmsprop": 3}


def optimizer_step_multi(kind: str, params: list, lr: float, hyper: float = 0.0, eps: float = 0.0) -> None:
    """params: list of (W, g, state) device tensors (state None for SGD)."""
    import ctypes as C
    n = len(params)
    arr = lambda idx: (C.c_void_p * n)(*[_p(p[idx]) if p[idx] is not None else None for p in params])
    sizes = (C.c_int64 * n)(*[p[0].numel() for p in params])
    _capi.call("cnhip_optimizer_step_multi", OPT[kind], n, arr(0), arr(1), arr(2), sizes, lr, hyper, eps,
               _stream())


def leaky_relu_forward(x, y, alpha: float) -> None:
    _capi.call("cnhip_leaky_relu_forward", _p(x), _p(y), x.numel(), alpha, _stream())


def leaky_relu_backward(x, dy, dx, alpha: float) -> None:
    _capi.call("cnhip_leaky_relu_backward", _p(x), _p(dy), _p(dx), x.numel(), alpha, _stream())


def softmax_forward(x, y, rows: int, length: int) -> None:
    _capi.call("cnhip_softmax_forward", _p(x), _p(y), rows, length, _stream())


def softmax_backward(y, dy, dx, rows: int, length: int) -> None:
    _capi.call("cnhip_softmax_backward", _p(y), _p(dy), _p(dx), rows, length, _stream())


def cce_forward(pred, t, probs, tu, loss, B: int, C: int, from_logits: bool, ls: float,
                reduction: str = "mean") -> None:
    _capi.call("cnhip_cce_forward", _p(pred), _p(t), _p(probs), _p(tu), _p(loss), B, C, int(from_logits),
               ls, _red(reduction), _stream())


def cce_backward(probs, tu, g, B: int, C: int, from_logits: bool, reduction: str = "mean") -> None:
    _capi.call("cnhip_cce_backward", _p(probs), _p(tu), _p(g), B, C, int(from_logits), _red(reduction),
               _stream())


def mae_forward(p, t, loss, reduction: str = "mean") -> None:
    _capi.call("cnhip_mae_forward", _p(p), _p(t), _p(loss), p.numel(), _red(reduction), _stream())


def mae_backward(p, t, g, reduction: str = "mean") -> None:
    _capi.call("cnhip_mae_backward", _p(p), _p(t), _p(g), p.numel(), _red(reduction), _stream())


def huber_forward(p, t, loss, delta: float, reduction: str = "mean") -> None:
    _capi.call("cnhip_huber_forward", _p(p), _p(t), _p(loss), p.numel(), delta, _red(reduction),
               _stream())


def huber_backward(p, t, g, delta: float, reduction: str = "mean") -> None:
    _capi.call("cnhip_huber_backward", _p(p), _p(t), _p(g), p.numel(), delta, _red(reduction),
               _stream())


def dropout_forward(x, y, mask, p: float, seed: int, offset: int = 0) -> None:
    _capi.call("cnhip_dropout_forward", _p(x), _p(y), _p(mask), x.numel(), p, seed, offset, _stream())


def dropout_backward(dy, mask, dx, p: float) -> None:
    _capi.call("cnhip_dropout_backward", _p(dy), _p(mask), _p(dx), dy.numel(), p, _stream())


def global_avgpool_forward(X, Y, N, C, H, W) -> None:
    _capi.call("cnhip_global_avgpool_forward", _p(X), _p(Y), N, C, H, W, _stream())


def global_avgpool_backward(dY, dX, N, C, H, W) -> None:
    _capi.call("cnhip_global_avgpool_backward", _p(dY), _p(dX), N, C, H, W, _stream())


def global_maxpool_forward(X, Y, ah, aw, N, C, H, W) -> None:
    _capi.call("cnhip_global_maxpool_forward", _p(X), _p(Y), _p(ah), _p(aw), N, C, H, W, _stream())


def global_maxpool_backward(dY, ah, aw, dX, N, C, H, W) -> None:
    _capi.call("cnhip_global_maxpool_backward", _p(dY), _p(ah), _p(aw), _p(dX), N, C, H, W, _stream())


def rnn_forward(X, W_ih, W_hh, b, Y, B, S, I, H) -> None:
    _capi.call("cnhip_rnn_forward", _p(X), _p(W_ih), _p(W_hh), _p(b), _p(Y), B, S, I, H, _stream())


def rnn_backward(X, W_ih, W_hh, Y, dY, gW_ih, gW_hh, gb, dX, B, S, I, H) -> None:
    _capi.call("cnhip_rnn_backward", *(_p(t) for t in (X, W_ih, W_hh, Y, dY, gW_ih, gW_hh, gb, dX)), B, S, I,
               H, _stream())

