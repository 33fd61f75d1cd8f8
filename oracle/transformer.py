"""Transformer-classifier train step composed from the CPU oracle's ops (test
infrastructure): Embedding -> blocks x [r = MHA(x,x,x) + x; h = BatchNorm(r
on [B*S, D]); y = Linear2(GELU(Linear1(h))) + h] -> MeanPool1D -> Linear ->
SoftmaxCE(mean) -> Adam, the harness composition of
benchmarks/transformer_benckmark.cpp:95-175 with the layers of
src/CppNet/layers/{embedding,attention,batch_norm,mean_pool1d}.cpp.
Embedding, MHA and BatchNorm grads are overwritten by their backward
(embedding.cpp:108, attention.cpp:505-508, batch_norm.cpp:353-385); Linear
grads are cleared by zero_grad and accumulated (linear.cpp:346-352)."""
from __future__ import annotations

import numpy as np

from oracle import fp, ip

_MEAN = 0


class OracleTransformer:
    def __init__(self, cfg, oracle):
        self.cfg, self.o = cfg, oracle
        D, nb = cfg.embed_dim, cfg.blocks
        self.rmean = [np.zeros(D, np.float32) for _ in range(nb)]
        self.rvar = [np.ones(D, np.float32) for _ in range(nb)]

    def set_params(self, params):
        self.params = [np.array(p, np.float32, copy=True) for p in params]
        self.grads = [np.zeros_like(p) for p in self.params]
        self.m = [np.zeros_like(p) for p in self.params]
        self.v = [np.zeros_like(p) for p in self.params]
        self.t = [0] * len(self.params)

    def get_params(self):
        return [p.copy() for p in self.params]

    def _blk(self, i):
        """parameter indices of block i: Wq, Wk, Wv, Wo, gamma, beta, W1, b1, W2, b2"""
        return list(range(1 + 10 * i, 11 + 10 * i))

    def step(self, ids, Y):
        o, cfg = self.o, self.cfg
        B, S, V, D, F, C = cfg.batch, cfg.seq_len, cfg.vocab, cfg.embed_dim, cfg.ffn, cfg.classes
        BS, P, G = B * S, self.params, self.grads
        ids = np.ascontiguousarray(ids, np.int32)
        Y = np.ascontiguousarray(Y, np.float32)
        for gr in G:
            gr[...] = 0.0
        x = np.zeros(BS * D, np.float32)
        assert o.cnref_embedding_forward(ip(ids), fp(P[0]), fp(x), B, S, V, D) == 0
        trace = []
        for i in range(cfg.blocks):
            q, k, v, wo, gam, bet, w1, b1, w2, b2 = (P[j] for j in self._blk(i))
            a, attn = np.zeros(BS * D, np.float32), np.zeros(B * S * S, np.float32)
            o.cnref_mha_forward(fp(x), fp(x), fp(x), fp(q), fp(k), fp(v), fp(wo), fp(a), fp(attn), B, S, D,
                                cfg.heads)
            r = a + x
            h, xh = np.zeros(BS * D, np.float32), np.zeros(BS * D, np.float32)
            bm, bv = np.zeros(D, np.float32), np.zeros(D, np.float32)
            o.cnref_batchnorm_forward(fp(r), fp(h), fp(xh), fp(gam), fp(bet), fp(self.rmean[i]),
                                      fp(self.rvar[i]), fp(bm), fp(bv), BS, D, 0.1, 1e-5)
            z1 = np.zeros(BS * F, np.float32)
            o.cnref_linear_forward(fp(h), fp(w1), fp(b1), fp(z1), BS, D, F)
            g1 = np.zeros_like(z1)
            o.cnref_gelu_forward(fp(z1), fp(g1), z1.size)
            z2 = np.zeros(BS * D, np.float32)
            o.cnref_linear_forward(fp(g1), fp(w2), fp(b2), fp(z2), BS, F, D)
            trace.append(dict(x=x, attn=attn, r=r, h=h, xh=xh, bm=bm, bv=bv, z1=z1, g1=g1))
            x = z2 + h
        pooled = np.zeros(B * D, np.float32)
        o.cnref_meanpool1d_forward(fp(x), fp(pooled), B, S, D)
        logits = np.zeros(B * C, np.float32)
        o.cnref_linear_forward(fp(pooled), fp(P[-2]), fp(P[-1]), fp(logits), B, D, C)
        sm, gl = np.zeros_like(logits), np.zeros_like(logits)
        loss = o.cnref_softmax_ce_forward(fp(logits), fp(Y), fp(sm), B, C, _MEAN)
        o.cnref_softmax_ce_backward(fp(sm), fp(Y), fp(gl), B, C, _MEAN)
        dp = np.zeros(B * D, np.float32)
        o.cnref_linear_backward(fp(pooled), fp(P[-2]), fp(gl), fp(G[-2]), fp(G[-1]), fp(dp), B, D, C, 1, 1)
        dy = np.zeros(BS * D, np.float32)
        o.cnref_meanpool1d_backward(fp(dp), fp(dy), B, S, D)
        keep = getattr(self, "keep", True)
        self.head_trace = dict(pooled=pooled, gl=gl)
        for i in reversed(range(cfg.blocks)):
            T = trace[i]
            iq, ik, iv, io, ig, ib, i1, ib1, i2, ib2 = self._blk(i)
            dg1 = np.zeros(BS * F, np.float32)
            o.cnref_linear_backward(fp(T["g1"]), fp(P[i2]), fp(dy), fp(G[i2]), fp(G[ib2]), fp(dg1), BS, F, D, 1, 1)
            dz1 = np.zeros_like(dg1)
            o.cnref_gelu_backward(fp(T["z1"]), fp(dg1), fp(dz1), dz1.size)
            dh = np.zeros(BS * D, np.float32)
            o.cnref_linear_backward(fp(T["h"]), fp(P[i1]), fp(dz1), fp(G[i1]), fp(G[ib1]), fp(dh), BS, D, F, 1, 1)
            gh = dh + dy
            dr = np.zeros(BS * D, np.float32)
            o.cnref_batchnorm_backward(fp(gh), fp(T["r"]), fp(T["xh"]), fp(P[ig]), fp(T["bm"]), fp(T["bv"]),
                                       fp(G[ig]), fp(G[ib]), fp(dr), BS, D, 1e-5)
            dxa = np.zeros(BS * D, np.float32)
            xx = T["x"]
            if keep:  # the operands of the weight-gradient contractions, for the tests' error bars
                T.update(dy=dy, dz1=dz1, gh=gh, dr=dr)
                for slot, name in ((1, "gQp"), (2, "gKp"), (3, "gVp"), (4, "ctx")):
                    T[name] = np.zeros(BS * D, np.float32)
                    o.cnref_set_trace(slot, fp(T[name]))
            o.cnref_mha_backward(fp(xx), fp(xx), fp(xx), fp(P[iq]), fp(P[ik]), fp(P[iv]), fp(P[io]),
                                 fp(T["attn"]), fp(dr), fp(G[iq]), fp(G[ik]), fp(G[iv]), fp(G[io]), fp(dxa),
                                 B, S, D, cfg.heads)
            for slot in (1, 2, 3, 4):
                o.cnref_set_trace(slot, None)
            dy = dxa + dr
        o.cnref_embedding_backward(ip(ids), fp(dy), fp(G[0]), B, S, V, D)
        self.head_trace.update(demb=dy, ids=ids)
        if getattr(self, "keep", True):  # per-step diagnostics; long runs turn them off
            self.last_grads = [gr.copy() for gr in G]
        self.trace = trace
        for kk, (p, gr) in enumerate(zip(P, G)):
            self.t[kk] += 1
            bc1 = o.cnref_bias_correction(cfg.beta1, self.t[kk])
            bc2 = o.cnref_bias_correction(cfg.beta2, self.t[kk])
            o.cnref_adam_step(fp(p), fp(gr), fp(self.m[kk]), fp(self.v[kk]), p.size, cfg.lr, cfg.beta1,
                              cfg.beta2, cfg.eps, bc1, bc2)
        return float(loss)
