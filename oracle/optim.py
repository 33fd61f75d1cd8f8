"""Per-parameter optimizer state and update of the oracle model compositions
(test infrastructure).  Each parameter keeps its own state and step count,
as the reference keys them by the weight pointer:
Adam (src/CppNet/optimizers/adam.cpp:98-133), SGD (sgd.cpp:54-68),
Momentum (momentum.cpp:81-104), Adagrad (adagrad.cpp:83-106) and RMSProp
(mrs_prop.cpp:83-106), each step through the oracle's C restatement."""
from __future__ import annotations

import numpy as np

from oracle import fp


class OracleOptimizer:
    def __init__(self, cfg, oracle, params):
        self.o = oracle
        self.kind = getattr(cfg, "optimizer", "adam")
        self.lr = cfg.lr
        self.beta1, self.beta2, self.eps = cfg.beta1, cfg.beta2, cfg.eps
        self.hyper = getattr(cfg, "opt_hyper", 0.9)
        self.opt_eps = getattr(cfg, "opt_eps", 1e-8)
        self.m = [np.zeros_like(p) for p in params]
        self.v = [np.zeros_like(p) for p in params]
        self.t = [0] * len(params)

    def step(self, params, grads):
        o = self.o
        for k, (p, g) in enumerate(zip(params, grads)):
            if self.kind == "adam":
                self.t[k] += 1
                bc1 = o.cnref_bias_correction(self.beta1, self.t[k])
                bc2 = o.cnref_bias_correction(self.beta2, self.t[k])
                o.cnref_adam_step(fp(p), fp(g), fp(self.m[k]), fp(self.v[k]), p.size, self.lr,
                                  self.beta1, self.beta2, self.eps, bc1, bc2)
            elif self.kind == "sgd":
                o.cnref_sgd_step(fp(p), fp(g), p.size, self.lr)
            elif self.kind == "momentum":
                o.cnref_momentum_step(fp(p), fp(g), fp(self.m[k]), p.size, self.lr, self.hyper)
            elif self.kind == "adagrad":
                o.cnref_adagrad_step(fp(p), fp(g), fp(self.m[k]), p.size, self.lr, self.opt_eps)
            elif self.kind == "rmsprop":
                o.cnref_rmsprop_step(fp(p), fp(g), fp(self.m[k]), p.size, self.lr, self.hyper,
                                     self.opt_eps)
            else:
                raise ValueError(f"unknown optimizer {self.kind!r}")
