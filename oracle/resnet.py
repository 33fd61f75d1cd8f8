"""Residual-network reference composed from the CPU oracle's ops (test
infrastructure).  The model is the reference's residual benchmark
(benchmarks/residual_benckmark.cpp:104-152):

  Linear(in, W) -> ReLU -> [Residual([Linear(w, W), Linear(W, w')], w, w') -> ReLU] x depth
  -> Linear(w_last, classes) -> SoftmaxCrossEntropy("mean"), Adam

with w = W for every block and w' = W except the last block's, which maps to
cfg.last_width (a projection shortcut when that differs from W,
residual.cpp:31-36).  The train step is the harness's (residual_benckmark.cpp:
186-196): zero_grad, forward, loss, backward, update; Linear grads accumulate
(linear.cpp:346-352).  Residual's forward/backward are cnref_residual_* (the
C restatement of residual.cpp:44-131)."""
from __future__ import annotations

import ctypes as C

import numpy as np

from oracle import fp
from oracle.optim import OracleOptimizer

_RED_MEAN = 0
_f = C.POINTER(C.c_float)


def _ptrs(arrs):
    return (_f * len(arrs))(*[fp(a) if a is not None else None for a in arrs])


def residual_forward(o, block_W, block_b, Wp, x, B, sizes):
    """y = block(x) + shortcut(x) and the block layers' outputs (cnref_residual_forward)."""
    n = len(block_W)
    acts = [np.empty(B * sizes[i + 1], np.float32) for i in range(n)]
    y = np.empty(B * sizes[-1], np.float32)
    o.cnref_residual_forward(n, (C.c_int64 * len(sizes))(*sizes), _ptrs(block_W), _ptrs(block_b), fp(Wp),
                             fp(x), _ptrs(acts), fp(y), B)
    return y, acts


def residual_backward(o, block_W, Wp, x, acts, dY, gW, gb, gWp, B, sizes):
    """dX, accumulating into gW[i], gb[i] and gWp (cnref_residual_backward)."""
    n = len(block_W)
    dX = np.empty(B * sizes[0], np.float32)
    o.cnref_residual_backward(n, (C.c_int64 * len(sizes))(*sizes), _ptrs(block_W), fp(Wp), fp(x), _ptrs(acts),
                              fp(dY), _ptrs(gW), _ptrs(gb), fp(gWp), fp(dX), B)
    return dX


def resnet_layout(cfg):
    """Parameter shapes in session order: proj W, b; per block fc_a W, b,
    fc_b W, b [, ResProj W]; head W, b.  Returns (shapes, block_sizes) with
    block_sizes[d] = (w_in, W, w_out)."""
    shapes = [(cfg.in_features, cfg.width), (cfg.width,)]
    blocks = []
    for d in range(cfg.depth):
        w_out = cfg.last_width if d + 1 == cfg.depth else cfg.width
        blocks.append((cfg.width, cfg.width, w_out))
        shapes += [(cfg.width, cfg.width), (cfg.width,), (cfg.width, w_out), (w_out,)]
        if w_out != cfg.width:
            shapes.append((cfg.width, w_out))
    w_last = blocks[-1][2] if blocks else cfg.width
    shapes += [(w_last, cfg.classes), (cfg.classes,)]
    return shapes, blocks


class OracleResNet:
    def __init__(self, cfg, oracle):
        self.cfg = cfg
        self.o = oracle
        self.shapes, self.blocks = resnet_layout(cfg)

    def set_params(self, params):
        self.params = [np.array(p, np.float32, copy=True) for p in params]
        self.grads = [np.zeros_like(p) for p in self.params]
        self.opt = OracleOptimizer(self.cfg, self.o, self.params)

    def get_params(self):
        return [p.copy() for p in self.params]

    def step(self, X, Y):
        o, cfg, B = self.o, self.cfg, self.cfg.batch
        P, G = self.params, self.grads
        for g in G:  # model.zero_grad()
            g[...] = 0.0
        X = np.ascontiguousarray(X, np.float32)
        Y = np.ascontiguousarray(Y, np.float32)
        # forward
        z0 = np.empty(B * cfg.width, np.float32)
        o.cnref_linear_forward(fp(X), fp(P[0]), fp(P[1]), fp(z0), B, cfg.in_features, cfg.width)
        h = np.empty_like(z0)
        o.cnref_relu_forward(fp(z0), fp(h), h.size)
        relu_out = [h]
        saved = []
        k = 2
        for (w_in, W, w_out) in self.blocks:
            idx = dict(Wa=k, ba=k + 1, Wb=k + 2, bb=k + 3, Wp=k + 4 if w_out != w_in else None)
            k += 5 if idx["Wp"] is not None else 4
            sizes = [w_in, W, w_out]
            Wp = P[idx["Wp"]] if idx["Wp"] is not None else None
            y, acts = residual_forward(o, [P[idx["Wa"]], P[idx["Wb"]]], [P[idx["ba"]], P[idx["bb"]]], Wp, h, B,
                                       sizes)
            saved.append((idx, sizes, h, acts))
            h = np.empty_like(y)
            o.cnref_relu_forward(fp(y), fp(h), h.size)
            relu_out.append(h)
        w_last = self.shapes[-2][0]
        out = np.empty(B * cfg.classes, np.float32)
        o.cnref_linear_forward(fp(h), fp(P[k]), fp(P[k + 1]), fp(out), B, w_last, cfg.classes)
        # loss
        sm, grad = np.empty_like(out), np.empty_like(out)
        loss = o.cnref_softmax_ce_forward(fp(out), fp(Y), fp(sm), B, cfg.classes, _RED_MEAN)
        o.cnref_softmax_ce_backward(fp(sm), fp(Y), fp(grad), B, cfg.classes, _RED_MEAN)
        # backward; trace[k] = (input x, output gradient dA, I, O) of the
        # Linear whose weight is parameter k (for the tests' magnitude bars)
        self.trace = {0: (X, None, cfg.in_features, cfg.width), k: (h, grad, w_last, cfg.classes)}
        dh = np.empty(B * w_last, np.float32)
        o.cnref_linear_backward(fp(h), fp(P[k]), fp(grad), fp(G[k]), fp(G[k + 1]), fp(dh), B, w_last,
                                cfg.classes, 1, 1)
        for bi in reversed(range(len(self.blocks))):
            idx, sizes, x_in, acts = saved[bi]
            dy = np.empty_like(dh)
            o.cnref_relu_backward(fp(relu_out[bi + 1]), fp(dh), fp(dy), dy.size)
            Wp = P[idx["Wp"]] if idx["Wp"] is not None else None
            gWp = G[idx["Wp"]] if idx["Wp"] is not None else None
            dh = residual_backward(o, [P[idx["Wa"]], P[idx["Wb"]]], Wp, x_in, acts, dy,
                                   [G[idx["Wa"]], G[idx["Wb"]]], [G[idx["ba"]], G[idx["bb"]]], gWp, B, sizes)
            da = np.empty(B * sizes[1], np.float32)  # gradient at fc_a's output: dy W_b^T
            o.cnref_gemm_f32(0, 1, B, sizes[1], sizes[2], 1.0, fp(dy), B, fp(P[idx["Wb"]]), sizes[1], 0.0, fp(da),
                             B, None, 0)
            self.trace[idx["Wa"]] = (x_in, da, sizes[0], sizes[1])
            self.trace[idx["Wb"]] = (acts[0], dy, sizes[1], sizes[2])
            if idx["Wp"] is not None:
                self.trace[idx["Wp"]] = (x_in, dy, sizes[0], sizes[2])
        dz0 = np.empty_like(dh)
        o.cnref_relu_backward(fp(relu_out[0]), fp(dh), fp(dz0), dz0.size)
        self.trace[0] = (X, dz0, cfg.in_features, cfg.width)
        o.cnref_linear_backward(fp(X), fp(P[0]), fp(dz0), fp(G[0]), fp(G[1]), None, B, cfg.in_features,
                                cfg.width, 1, 1)
        self.opt.step(P, G)
        self.last_grads = [g.copy() for g in G]
        return float(loss)
