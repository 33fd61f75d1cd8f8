"""CNN train step composed from the CPU oracle's ops (test infrastructure):
conv blocks (Conv2D -> ReLU -> MaxPool2D), Flatten, Linear, softmax-CE and
Adam, in the order of the reference harness (benchmarks/cnn_benckmark.cpp:
219-274).  Conv grads are overwritten each backward (conv2d.cpp:149-152);
the Linear grads are cleared by zero_grad and accumulated (linear.cpp:346-352)."""
from __future__ import annotations

import numpy as np

from oracle import fp, ip


class OracleCNN:
    def __init__(self, cfg, oracle):
        self.cfg, self.o = cfg, oracle

    def set_params(self, params):
        self.params = [np.array(p, np.float32, copy=True) for p in params]
        self.grads = [np.zeros_like(p) for p in self.params]
        self.m = [np.zeros_like(p) for p in self.params]
        self.v = [np.zeros_like(p) for p in self.params]
        self.t = [0] * len(self.params)

    def get_params(self):
        return [p.copy() for p in self.params]

    def step(self, X, Y):
        o, cfg = self.o, self.cfg
        N, C, H, W = cfg.input_shape
        x = np.ascontiguousarray(X, np.float32)
        cache = []
        for i, (ic, oc, k, s, p) in enumerate(cfg.convs):
            HO, WO = (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1
            z = np.empty(N * oc * HO * WO, np.float32)
            o.cnref_conv2d_forward(fp(x), fp(self.params[2 * i]), fp(self.params[2 * i + 1]), fp(z),
                                   N, ic, H, W, oc, k, s, p)
            a = np.empty_like(z)
            o.cnref_relu_forward(fp(z), fp(a), z.size)
            PH, PW = (HO - cfg.pool) // cfg.pool + 1, (WO - cfg.pool) // cfg.pool + 1
            y = np.empty(N * oc * PH * PW, np.float32)
            idx = np.empty(N * oc * PH * PW, np.int32)
            o.cnref_maxpool2d_forward(fp(a), fp(y), ip(idx), N, oc, HO, WO, cfg.pool, cfg.pool)
            cache.append((x, (ic, oc, k, s, p, H, W, HO, WO), a, idx, z))
            x, C, H, W = y, oc, PH, PW
        F = C * H * W  # Flatten: the same ColMajor buffer
        L = len(cfg.convs)
        logits = np.empty(N * cfg.classes, np.float32)
        o.cnref_linear_forward(fp(x), fp(self.params[2 * L]), fp(self.params[2 * L + 1]), fp(logits),
                               N, F, cfg.classes)
        sm, g = np.empty_like(logits), np.empty_like(logits)
        Yc = np.ascontiguousarray(Y, np.float32)
        loss = o.cnref_softmax_ce_forward(fp(logits), fp(Yc), fp(sm), N, cfg.classes, 0)
        o.cnref_softmax_ce_backward(fp(sm), fp(Yc), fp(g), N, cfg.classes, 0)
        self.grads[2 * L][...] = 0.0
        self.grads[2 * L + 1][...] = 0.0
        dx = np.empty(N * F, np.float32)
        o.cnref_linear_backward(fp(x), fp(self.params[2 * L]), fp(g), fp(self.grads[2 * L]),
                                fp(self.grads[2 * L + 1]), fp(dx), N, F, cfg.classes, 1, 1)
        self.trace = []
        for i in reversed(range(L)):
            xin, (ic, oc, k, s, p, H, W, HO, WO), a, idx, z = cache[i]
            gpool = dx.copy()
            da = np.empty(N * oc * HO * WO, np.float32)
            o.cnref_maxpool2d_backward(fp(dx), ip(idx), fp(da), N, oc, HO, WO, cfg.pool, cfg.pool)
            dz = np.empty_like(da)
            o.cnref_relu_backward(fp(a), fp(da), fp(dz), da.size)
            dxi = np.empty_like(xin)
            o.cnref_conv2d_backward(fp(xin), fp(self.params[2 * i]), fp(dz), fp(self.grads[2 * i]),
                                    fp(self.grads[2 * i + 1]), fp(dxi), N, ic, H, W, oc, k, s, p)
            self.trace.insert(0, dict(x=xin, z=z, a=a, idx=idx, gpool=gpool, da=da, dz=dz,
                                      dims=(ic, oc, k, s, p, H, W, HO, WO)))
            dx = dxi
        self.fc_trace = dict(x=x, g=g, F=F)
        if getattr(self, "keep", True):  # per-step diagnostics; long runs turn them off
            self.last_grads = [gr.copy() for gr in self.grads]
        for k_, (p_, g_) in enumerate(zip(self.params, self.grads)):
            self.t[k_] += 1
            bc1 = o.cnref_bias_correction(cfg.beta1, self.t[k_])
            bc2 = o.cnref_bias_correction(cfg.beta2, self.t[k_])
            o.cnref_adam_step(fp(p_), fp(g_), fp(self.m[k_]), fp(self.v[k_]), p_.size, cfg.lr,
                              cfg.beta1, cfg.beta2, cfg.eps, bc1, bc2)
        return float(loss)
