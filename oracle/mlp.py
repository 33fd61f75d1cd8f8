"""Model-level reference composed from the CPU oracle's ops (test
infrastructure).  Runs the reference harness's train step
(benchmarks/mlp_benchmark.cpp:166-175): zero_grad, forward, loss forward and
backward, backward, Adam update per parameter with per-key step counts
(adam.cpp:98-133).  Linear grads accumulate (linear.cpp:346-352) and are
cleared by zero_grad (models.cpp:72-78)."""
from __future__ import annotations

import numpy as np

from oracle import fp
from oracle.optim import OracleOptimizer

_RED_MEAN = 0


class OracleMLP:
    def __init__(self, cfg, oracle):
        self.cfg = cfg
        self.o = oracle
        self.sizes = cfg.sizes
        self.params = None
        self.grads = None
        self.opt = None
        self.keep = True  # keep the per-step diagnostics (trace, last_grads); long runs turn it off

    def set_params(self, params):
        self.params = [np.array(p, np.float32, copy=True) for p in params]
        self.grads = [np.zeros_like(p) for p in self.params]
        self.opt = OracleOptimizer(self.cfg, self.o, self.params)

    def get_params(self):
        return [p.copy() for p in self.params]

    def _act(self, name, x):
        y = np.empty_like(x)
        if name == "leaky_relu":  # leacky_relu.hpp default alpha
            self.o.cnref_leaky_relu_forward(fp(x), fp(y), x.size, 0.01)
        elif name == "softmax":  # over the features of each of the B rows
            self.o.cnref_softmax_forward(fp(x), fp(y), self.cfg.batch, x.size // self.cfg.batch)
        elif name == "relu":
            self.o.cnref_relu_forward(fp(x), fp(y), x.size)
        elif name == "sigmoid":
            self.o.cnref_sigmoid_forward(fp(x), fp(y), x.size)
        elif name == "tanh":
            self.o.cnref_tanh_forward(fp(x), fp(y), x.size)
        else:
            return x
        return y

    def _act_bwd(self, name, y, g, z=None):
        if name == "none":
            return g
        dx = np.empty_like(g)
        if name == "leaky_relu":  # reads the cached input (leacky_relu.cpp:127-160)
            self.o.cnref_leaky_relu_backward(fp(z), fp(g), fp(dx), g.size, 0.01)
            return dx
        if name == "softmax":
            self.o.cnref_softmax_backward(fp(y), fp(g), fp(dx), self.cfg.batch, g.size // self.cfg.batch)
            return dx
        getattr(self.o, f"cnref_{name}_backward")(fp(y), fp(g), fp(dx), g.size)
        return dx

    def step(self, X, Y):
        o, B, cfg = self.o, self.cfg.batch, self.cfg
        X = np.ascontiguousarray(X, np.float32)
        Y = np.ascontiguousarray(Y, np.float32)
        for g in self.grads:  # model.zero_grad()
            g[...] = 0.0
        nl = len(self.sizes) - 1
        inputs, outs, acts, pre = [], [], [], []
        h = X
        for i in range(nl):
            I, O = self.sizes[i], self.sizes[i + 1]
            z = np.empty(B * O, np.float32)
            o.cnref_linear_forward(fp(h), fp(self.params[2 * i]), fp(self.params[2 * i + 1]),
                                   fp(z), B, I, O)
            inputs.append(h)
            pre.append(z)
            act = cfg.hidden_act if i + 1 < nl else cfg.out_act
            h = self._act(act, z)
            acts.append(act)
            outs.append(h)
        out = h
        O = self.sizes[-1]
        grad = np.empty_like(out)
        if cfg.loss == "bce":
            loss = o.cnref_bce_forward(fp(out), fp(Y), out.size, _RED_MEAN)
            o.cnref_bce_backward(fp(out), fp(Y), fp(grad), out.size, _RED_MEAN)
        elif cfg.loss == "softmax_ce":
            sm = np.empty_like(out)
            loss = o.cnref_softmax_ce_forward(fp(out), fp(Y), fp(sm), B, O, _RED_MEAN)
            o.cnref_softmax_ce_backward(fp(sm), fp(Y), fp(grad), B, O, _RED_MEAN)
        elif cfg.loss == "cce":  # from logits, no smoothing
            sm, tu = np.empty_like(out), np.empty_like(out)
            loss = o.cnref_cce_forward(fp(out), fp(Y), fp(sm), fp(tu), B, O, 1, 0.0, _RED_MEAN)
            o.cnref_cce_backward(fp(sm), fp(tu), fp(grad), B, O, 1, _RED_MEAN)
        elif cfg.loss == "mae":
            loss = o.cnref_mae_forward(fp(out), fp(Y), out.size, _RED_MEAN)
            o.cnref_mae_backward(fp(out), fp(Y), fp(grad), out.size, _RED_MEAN)
        elif cfg.loss == "huber":  # delta 1
            loss = o.cnref_huber_forward(fp(out), fp(Y), out.size, 1.0, _RED_MEAN)
            o.cnref_huber_backward(fp(out), fp(Y), fp(grad), out.size, 1.0, _RED_MEAN)
        else:
            loss = o.cnref_mse_forward(fp(out), fp(Y), out.size, _RED_MEAN)
            o.cnref_mse_backward(fp(out), fp(Y), fp(grad), out.size, _RED_MEAN)
        # per layer, for the tests' tolerances: layer input x, pre-activation z,
        # gradient w.r.t. the activation output dH and w.r.t. z (dA)
        self.trace = [None] * nl
        for i in reversed(range(nl)):
            I, O = self.sizes[i], self.sizes[i + 1]
            dH = grad
            grad = self._act_bwd(acts[i], outs[i], grad, pre[i])
            if self.keep:
                self.trace[i] = dict(x=inputs[i], z=pre[i], dH=dH.copy(), dA=grad.copy(), act=acts[i])
            dX = np.empty(B * I, np.float32)
            o.cnref_linear_backward(fp(inputs[i]), fp(self.params[2 * i]), fp(grad),
                                    fp(self.grads[2 * i]), fp(self.grads[2 * i + 1]), fp(dX), B, I,
                                    O, 1, 1)
            grad = dX
        self.opt.step(self.params, self.grads)  # model.update(optimizer, lr)
        if self.keep:
            self.last_grads = [g.copy() for g in self.grads]
        return float(loss)
