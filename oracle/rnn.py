"""Sequence-regressor train step composed from the CPU oracle's ops (test
infrastructure): LSTM, GRU or Elman RNN over the sequence, the last hidden
state, Linear, MSE(mean), Adam or the configured optimizer -- the reference
harness's loop
(benchmarks/sequence_benckmark.cpp:149-177).  Recurrent grads are
overwritten by each backward (lstm.cpp:158-160); the Linear grads are
cleared by zero_grad and accumulated (linear.cpp:346-352)."""
from __future__ import annotations

import numpy as np

from oracle import fp
from oracle.optim import OracleOptimizer


class OracleSeqRegressor:
    def __init__(self, cfg, oracle):
        self.cfg, self.o = cfg, oracle

    def set_params(self, params):
        self.params = [np.array(p, np.float32, copy=True) for p in params]
        self.grads = [np.zeros_like(p) for p in self.params]
        self.opt = OracleOptimizer(self.cfg, self.o, self.params)

    def get_params(self):
        return [p.copy() for p in self.params]

    def step(self, X, Y):
        o, cfg = self.o, self.cfg
        B, S, I, H, O = cfg.batch, cfg.seq_len, cfg.input_size, cfg.hidden, cfg.out_features
        BS = B * S
        X = np.ascontiguousarray(X, np.float32)
        Wih, Whh, b, W, bb = self.params
        Yseq = np.zeros(BS * H, np.float32)
        if cfg.cell == "lstm":
            gates = np.zeros(BS * 4 * H, np.float32)
            c, tc = np.zeros(BS * H, np.float32), np.zeros(BS * H, np.float32)
            o.cnref_lstm_forward(fp(X), fp(Wih), fp(Whh), fp(b), fp(Yseq), fp(gates), fp(c), fp(tc),
                                 B, S, I, H)
        elif cfg.cell == "rnn":
            o.cnref_rnn_forward(fp(X), fp(Wih), fp(Whh), fp(b), fp(Yseq), B, S, I, H)
        else:
            gates, rh = np.zeros(BS * 3 * H, np.float32), np.zeros(BS * H, np.float32)
            o.cnref_gru_forward(fp(X), fp(Wih), fp(Whh), fp(b), fp(Yseq), fp(gates), fp(rh), B, S, I, H)
        # last hidden state [B, H] = Y[:, S-1, :]
        hT = np.ascontiguousarray(Yseq.reshape(H, S, B)[:, S - 1, :]).ravel()
        pred = np.zeros(B * O, np.float32)
        o.cnref_linear_forward(fp(hT), fp(W), fp(bb), fp(pred), B, H, O)
        Yt = np.ascontiguousarray(Y, np.float32)
        loss = o.cnref_mse_forward(fp(pred), fp(Yt), pred.size, 0)
        g = np.zeros_like(pred)
        o.cnref_mse_backward(fp(pred), fp(Yt), fp(g), pred.size, 0)
        self.grads[3][...] = 0.0
        self.grads[4][...] = 0.0
        dh = np.zeros(B * H, np.float32)
        o.cnref_linear_backward(fp(hT), fp(W), fp(g), fp(self.grads[3]), fp(self.grads[4]), fp(dh), B,
                                H, O, 1, 1)
        dY = np.zeros((H, S, B), np.float32)
        dY[:, S - 1, :] = dh.reshape(H, B)
        dY = dY.ravel()
        dX = np.zeros_like(X)
        keep = getattr(self, "keep", True)
        # the gate pre-activation gradients of every timestep, for the tests' error bars
        dpre = np.zeros(BS * {"lstm": 4, "gru": 3, "rnn": 1}[cfg.cell] * H, np.float32) if keep else None
        o.cnref_set_trace(0, fp(dpre))
        if cfg.cell == "lstm":
            o.cnref_lstm_backward(fp(X), fp(Wih), fp(Whh), fp(Yseq), fp(gates), fp(c), fp(tc), fp(dY),
                                  fp(self.grads[0]), fp(self.grads[1]), fp(self.grads[2]), fp(dX),
                                  B, S, I, H)
        elif cfg.cell == "rnn":
            o.cnref_rnn_backward(fp(X), fp(Wih), fp(Whh), fp(Yseq), fp(dY), fp(self.grads[0]),
                                 fp(self.grads[1]), fp(self.grads[2]), fp(dX), B, S, I, H)
        else:
            o.cnref_gru_backward(fp(X), fp(Wih), fp(Whh), fp(Yseq), fp(gates), fp(rh), fp(dY),
                                 fp(self.grads[0]), fp(self.grads[1]), fp(self.grads[2]), fp(dX),
                                 B, S, I, H)
        o.cnref_set_trace(0, None)
        if keep:  # per-step diagnostics; long runs turn them off
            self.last_grads = [gr.copy() for gr in self.grads]
        self.trace = dict(X=X, Yseq=Yseq, hT=hT, g=g, dh=dh, dpre=dpre,
                          rh=rh if cfg.cell == "gru" else None)
        self.opt.step(self.params, self.grads)
        return float(loss)
