"""Pins the oracle's restatements of the reference's device ops off the
BASELINE configs (oracle/cnref_extra.cpp; CPU only, no GPU).

Each function is checked against (1) the known answers of the reference's own
tests (tests/golden/known_answers.json) and (2) what the mathematics fixes
independently of the oracle's loops: float64 torch autograd on logical
(row-major) tensors for forward values and gradients, and closed forms of the
optimizer recurrences under a constant gradient (geometric series), which a
wrong sign, a dropped term or an index slip in the ColMajor loops fails.
"""
import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle_lib import close, colmajor, fp, from_colmajor

GOLD = json.loads((Path(__file__).parent / "golden" / "known_answers.json").read_text())["cases"]


def _cases(op):
    return [c for c in GOLD if c["op"] == op]


def ip(a):
    import ctypes as C
    return a.ctypes.data_as(C.POINTER(C.c_int32))


def _cm(a):
    return colmajor(np.asarray(a, np.float32))


# ---------------------------------------------------------------- known answers
@pytest.mark.parametrize("case", _cases("leaky_relu_forward"), ids=lambda c: c["source"])
def test_known_leaky_relu_forward(oracle, case):
    x = _cm(case["X"])
    y = np.zeros_like(x)
    oracle.cnref_leaky_relu_forward(fp(x), fp(y), x.size, case["alpha"])
    assert close(y, _cm(case["expected"]), 0, case["tol"])[0]


@pytest.mark.parametrize("case", _cases("leaky_relu_backward"), ids=lambda c: c["source"])
def test_known_leaky_relu_backward(oracle, case):
    x, dy = _cm(case["X"]), _cm(case["dY"])
    dx = np.zeros_like(x)
    oracle.cnref_leaky_relu_backward(fp(x), fp(dy), fp(dx), x.size, case["alpha"])
    assert close(dx, _cm(case["expected"]), 0, case["tol"])[0]


@pytest.mark.parametrize("case", _cases("softmax_forward"), ids=lambda c: c["source"])
def test_known_softmax_forward(oracle, case):
    X = np.asarray(case["X"], np.float32)
    x = _cm(X)
    y = np.zeros_like(x)
    oracle.cnref_softmax_forward(fp(x), fp(y), X.shape[0], X.shape[1])
    assert close(y, _cm(case["expected"]), 0, case["tol"])[0]


@pytest.mark.parametrize("case", _cases("softmax_backward_constant"), ids=lambda c: c["source"])
def test_known_softmax_backward(oracle, case):
    X = np.asarray(case["X"], np.float32)
    x, dy = _cm(X), _cm(case["dY"])
    y, dx = np.zeros_like(x), np.zeros_like(x)
    oracle.cnref_softmax_forward(fp(x), fp(y), X.shape[0], X.shape[1])
    oracle.cnref_softmax_backward(fp(y), fp(dy), fp(dx), X.shape[0], X.shape[1])
    assert close(dx, _cm(case["expected"]), 0, case["tol"])[0]


def test_known_mae_and_huber(oracle):
    for c in _cases("mae_forward"):
        p, t = _cm(c["P"]), _cm(c["T"])
        assert abs(oracle.cnref_mae_forward(fp(p), fp(t), p.size, 0) - c["expected"]) <= c["tol"]
    for c in _cases("huber_forward"):
        p, t = _cm(c["P"]), _cm(c["T"])
        assert abs(oracle.cnref_huber_forward(fp(p), fp(t), p.size, c["delta"], 0) - c["expected"]) <= c["tol"]


def test_known_global_pools(oracle):
    for c in _cases("global_avgpool_forward") + _cases("global_maxpool_forward"):
        X = np.asarray(c["X"], np.float32)
        N, Cc, H, W = X.shape
        x, y = _cm(X), np.zeros(N * Cc, np.float32)
        if c["op"] == "global_avgpool_forward":
            oracle.cnref_global_avgpool_forward(fp(x), fp(y), N, Cc, H, W)
        else:
            ah, aw = np.zeros(N * Cc, np.int32), np.zeros(N * Cc, np.int32)
            oracle.cnref_global_maxpool_forward(fp(x), fp(y), ip(ah), ip(aw), N, Cc, H, W)
        assert close(y, _cm(c["expected"]), 0, c["tol"])[0]
    c = _cases("global_avgpool_backward")[0]
    N, Cc, H, W = c["shape"]
    dy, dx = _cm(c["dY"]), np.zeros(N * Cc * H * W, np.float32)
    oracle.cnref_global_avgpool_backward(fp(dy), fp(dx), N, Cc, H, W)
    assert close(dx, np.full_like(dx, c["expected_all"]), 0, c["tol"])[0]
    c = _cases("global_maxpool_backward")[0]
    X = np.asarray(c["X"], np.float32)
    N, Cc, H, W = X.shape
    x, y = _cm(X), np.zeros(N * Cc, np.float32)
    ah, aw = np.zeros(N * Cc, np.int32), np.zeros(N * Cc, np.int32)
    oracle.cnref_global_maxpool_forward(fp(x), fp(y), ip(ah), ip(aw), N, Cc, H, W)
    dx = np.full(x.size, 9.0, np.float32)
    oracle.cnref_global_maxpool_backward(fp(_cm(c["dY"])), ip(ah), ip(aw), fp(dx), N, Cc, H, W)
    assert close(dx, _cm(c["expected"]), 0, c["tol"])[0]


def test_known_dropout_scale(oracle):
    c = _cases("dropout_scale")[0]
    x = np.full(16, c["x"], np.float32)
    mask = np.tile(np.array([1, 0], np.float32), 8)
    y = np.zeros_like(x)
    scale = np.float32(1.0) / (np.float32(1.0) - np.float32(c["p"]))
    oracle.cnref_dropout_apply(fp(x), fp(mask), fp(y), x.size, float(scale))
    assert np.all(y[mask == 1] == np.float32(c["expected_kept"])) and np.all(y[mask == 0] == 0)


# ---------------------------------------------------------------- autograd (float64)
def test_leaky_relu_vs_autograd(oracle):
    rng = np.random.default_rng(1)
    X = rng.standard_normal((37, 11)).astype(np.float32)
    dY = rng.standard_normal((37, 11)).astype(np.float32)
    for alpha in (0.01, 0.3):
        xt = torch.tensor(X, dtype=torch.float64, requires_grad=True)
        yt = torch.nn.functional.leaky_relu(xt, alpha)
        yt.backward(torch.tensor(dY, dtype=torch.float64))
        x, dy = _cm(X), _cm(dY)
        y, dx = np.zeros_like(x), np.zeros_like(x)
        oracle.cnref_leaky_relu_forward(fp(x), fp(y), x.size, alpha)
        oracle.cnref_leaky_relu_backward(fp(x), fp(dy), fp(dx), x.size, alpha)
        assert close(y, colmajor(yt.detach().numpy()), 1e-6, 1e-7)[0]
        assert close(dx, colmajor(xt.grad.numpy()), 1e-6, 1e-7)[0]


@pytest.mark.parametrize("shape", [(9, 7), (2, 3, 4, 5), (5, 1)])
def test_softmax_last_dim_vs_autograd(oracle, shape):
    """2-D [B, F] and 4-D tensors: softmax over the last dimension, whose
    ColMajor stride is the product of the others."""
    rng = np.random.default_rng(sum(shape))
    X = (rng.standard_normal(shape) * 3).astype(np.float32)
    dY = rng.standard_normal(shape).astype(np.float32)
    xt = torch.tensor(X, dtype=torch.float64, requires_grad=True)
    yt = torch.softmax(xt, dim=-1)
    yt.backward(torch.tensor(dY, dtype=torch.float64))
    L = shape[-1]
    R = int(np.prod(shape)) // L
    x, dy = colmajor(X), colmajor(dY)
    y, dx = np.zeros_like(x), np.zeros_like(x)
    oracle.cnref_softmax_forward(fp(x), fp(y), R, L)
    oracle.cnref_softmax_backward(fp(y), fp(dy), fp(dx), R, L)
    assert close(y, colmajor(yt.detach().numpy()), 1e-5, 1e-7)[0]
    assert close(dx, colmajor(xt.grad.numpy()), 1e-4, 1e-6)[0]


@pytest.mark.parametrize("from_logits,ls,reduction", [(1, 0.0, 0), (1, 0.1, 0), (0, 0.0, 0), (0, 0.2, 1)])
def test_cce_vs_autograd(oracle, from_logits, ls, reduction):
    rng = np.random.default_rng(from_logits * 10 + int(ls * 10) + reduction)
    B, C = 13, 6
    labels = rng.integers(0, C, B)
    T = np.eye(C, dtype=np.float32)[labels]
    if from_logits:
        P = (rng.standard_normal((B, C)) * 2).astype(np.float32)
    else:
        P = rng.dirichlet(np.ones(C), B).astype(np.float32)
    pt = torch.tensor(P, dtype=torch.float64, requires_grad=True)
    Tt = torch.tensor(T, dtype=torch.float64) * (1 - ls) + ls / C if ls > 0 else torch.tensor(T, dtype=torch.float64)
    probs = torch.softmax(pt, dim=1) if from_logits else pt
    loss = -(Tt * torch.log(probs.clamp(1e-15, 1.0))).sum()
    if reduction == 0:
        loss = loss / B
    loss.backward()
    p, t = colmajor(P), colmajor(T)
    sm, tu, g = np.zeros_like(p), np.zeros_like(p), np.zeros_like(p)
    got = oracle.cnref_cce_forward(fp(p), fp(t), fp(sm), fp(tu), B, C, from_logits, ls, reduction)
    oracle.cnref_cce_backward(fp(sm), fp(tu), fp(g), B, C, from_logits, reduction)
    assert abs(got - loss.item()) <= 1e-5 * max(1.0, abs(loss.item()))
    # from_logits: the reference's gradient is d loss / d logits; for
    # probabilities it is d loss / d p (the clip is inactive here)
    assert close(g, colmajor(pt.grad.numpy()), 1e-5, 1e-7)[0]
    assert close(tu, colmajor(Tt.numpy()), 1e-7, 1e-8)[0]


def test_mae_huber_vs_autograd(oracle):
    rng = np.random.default_rng(3)
    P = (rng.standard_normal((20, 7)) * 2).astype(np.float32)
    T = (rng.standard_normal((20, 7)) * 2).astype(np.float32)
    p, t = colmajor(P), colmajor(T)
    for reduction in (0, 1):
        pt = torch.tensor(P, dtype=torch.float64, requires_grad=True)
        l1 = (pt - torch.tensor(T, dtype=torch.float64)).abs()
        l1 = l1.mean() if reduction == 0 else l1.sum()
        l1.backward()
        g = np.zeros_like(p)
        assert abs(oracle.cnref_mae_forward(fp(p), fp(t), p.size, reduction) - l1.item()) <= 1e-5 * abs(l1.item())
        oracle.cnref_mae_backward(fp(p), fp(t), fp(g), p.size, reduction)
        assert close(g, colmajor(pt.grad.numpy()), 1e-6, 1e-9)[0]
        for delta in (0.5, 1.0, 2.5):
            pt = torch.tensor(P, dtype=torch.float64, requires_grad=True)
            h = torch.nn.functional.huber_loss(pt, torch.tensor(T, dtype=torch.float64), reduction="sum",
                                               delta=delta)
            h = h / P.size if reduction == 0 else h
            h.backward()
            g = np.zeros_like(p)
            got = oracle.cnref_huber_forward(fp(p), fp(t), p.size, delta, reduction)
            assert abs(got - h.item()) <= 1e-5 * abs(h.item())
            oracle.cnref_huber_backward(fp(p), fp(t), fp(g), p.size, delta, reduction)
            assert close(g, colmajor(pt.grad.numpy()), 1e-6, 1e-9)[0]


@pytest.mark.parametrize("N,C,H,W", [(3, 4, 5, 6), (1, 1, 1, 1), (8, 2, 3, 3)])
def test_global_pools_vs_autograd(oracle, N, C, H, W):
    rng = np.random.default_rng(N * C + H * W)
    X = rng.integers(-4, 5, (N, C, H, W)).astype(np.float32)  # ties: first max (h-major) wins
    X += rng.standard_normal(X.shape).astype(np.float32) * (rng.random(X.shape) < 0.5)
    dY = rng.standard_normal((N, C)).astype(np.float32)
    xt = torch.tensor(X, dtype=torch.float64, requires_grad=True)
    xt.mean(dim=(2, 3)).backward(torch.tensor(dY, dtype=torch.float64))
    x = colmajor(X)
    y, dx = np.zeros(N * C, np.float32), np.zeros_like(x)
    oracle.cnref_global_avgpool_forward(fp(x), fp(y), N, C, H, W)
    oracle.cnref_global_avgpool_backward(fp(colmajor(dY)), fp(dx), N, C, H, W)
    assert close(y, colmajor(X.astype(np.float64).mean(axis=(2, 3))), 1e-5, 1e-6)[0]
    assert close(dx, colmajor(xt.grad.numpy()), 1e-6, 1e-8)[0]
    # max: value, the first (h-major) maximum's position, gradient routing
    ah, aw = np.zeros(N * C, np.int32), np.zeros(N * C, np.int32)
    oracle.cnref_global_maxpool_forward(fp(x), fp(y), ip(ah), ip(aw), N, C, H, W)
    flat = X.reshape(N, C, H * W)
    first = flat.argmax(axis=2)  # numpy: first occurrence in h-major order
    np.testing.assert_array_equal(y, colmajor(flat.max(axis=2)))
    np.testing.assert_array_equal(ah, colmajor((first // W).astype(np.int32)))
    np.testing.assert_array_equal(aw, colmajor((first % W).astype(np.int32)))
    dx = np.full_like(x, 5.0)
    oracle.cnref_global_maxpool_backward(fp(colmajor(dY)), ip(ah), ip(aw), fp(dx), N, C, H, W)
    want = np.zeros((N, C, H * W), np.float32)
    want[np.arange(N)[:, None], np.arange(C)[None, :], first] = dY
    np.testing.assert_array_equal(dx, colmajor(want.reshape(N, C, H, W)))


@pytest.mark.parametrize("B,S,I,H", [(3, 5, 4, 6), (1, 1, 2, 3), (4, 7, 3, 5)])
def test_rnn_vs_autograd(oracle, B, S, I, H):
    """Elman RNN (rnn.cpp): h_t = tanh(x_t W_ih + h_{t-1} W_hh + b), h_0 = 0,
    full sequence out; BPTT gradients of sum(out * dY)."""
    rng = np.random.default_rng(B * 100 + S * 10 + I + H)
    X = rng.standard_normal((B, S, I)).astype(np.float32)
    Wih = (rng.standard_normal((I, H)) * 0.5).astype(np.float32)
    Whh = (rng.standard_normal((H, H)) * 0.5).astype(np.float32)
    b = (rng.standard_normal(H) * 0.1).astype(np.float32)
    dY = rng.standard_normal((B, S, H)).astype(np.float32)
    t = [torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (X, Wih, Whh, b)]
    h = torch.zeros(B, H, dtype=torch.float64)
    outs = []
    for s in range(S):
        h = torch.tanh(t[0][:, s, :] @ t[1] + h @ t[2] + t[3])
        outs.append(h)
    Y = torch.stack(outs, dim=1)
    Y.backward(torch.tensor(dY, dtype=torch.float64))
    x, y = colmajor(X), np.zeros(B * S * H, np.float32)
    oracle.cnref_rnn_forward(fp(x), fp(colmajor(Wih)), fp(colmajor(Whh)), fp(b), fp(y), B, S, I, H)
    assert close(y, colmajor(Y.detach().numpy()), 1e-5, 1e-6)[0]
    gWih, gWhh, gb = np.zeros(I * H, np.float32), np.zeros(H * H, np.float32), np.zeros(H, np.float32)
    dx = np.zeros_like(x)
    oracle.cnref_rnn_backward(fp(x), fp(colmajor(Wih)), fp(colmajor(Whh)), fp(y), fp(colmajor(dY)),
                              fp(gWih), fp(gWhh), fp(gb), fp(dx), B, S, I, H)
    for got, want in ((gWih, t[1].grad), (gWhh, t[2].grad), (gb, t[3].grad), (dx, t[0].grad)):
        assert close(got, colmajor(want.numpy()), 1e-4, 1e-5)[0]


# ---------------------------------------------------------------- optimizers: closed forms
def test_optimizers_constant_gradient_closed_forms(oracle):
    """Under a constant gradient g the recurrences have closed forms:
    SGD       W_k = W_0 - k lr g
    Momentum  v_k = -lr g (1 - mu^k) / (1 - mu),  W_k = W_0 + sum_i v_i
    Adagrad   acc_k = k g^2,  W_k = W_0 - sum_i lr g / (sqrt(i) |g| + eps)
    RMSProp   s_k = (1 - rho^k) g^2,  W_k = W_0 - sum_i lr g / (sqrt(1 - rho^i) |g| + eps)."""
    g = np.array([0.5, -1.25, 3.0, -0.01, 2e-4], np.float32)
    W0 = np.array([1.0, -2.0, 0.25, 4.0, -0.5], np.float32)
    lr, mu, eps, rho, K = 0.05, 0.9, 1e-8, 0.9, 12
    g64, W64 = g.astype(np.float64), W0.astype(np.float64)
    Ws = [W0.copy() for _ in range(4)]
    st = [np.zeros_like(g) for _ in range(3)]
    for _ in range(K):
        oracle.cnref_sgd_step(fp(Ws[0]), fp(g), g.size, lr)
        oracle.cnref_momentum_step(fp(Ws[1]), fp(g), fp(st[0]), g.size, lr, mu)
        oracle.cnref_adagrad_step(fp(Ws[2]), fp(g), fp(st[1]), g.size, lr, eps)
        oracle.cnref_rmsprop_step(fp(Ws[3]), fp(g), fp(st[2]), g.size, lr, rho, eps)
    want = [W64 - K * lr * g64,
            W64 + sum(-lr * g64 * (1 - mu ** i) / (1 - mu) for i in range(1, K + 1)),
            W64 - sum(lr * g64 / (math.sqrt(i) * np.abs(g64) + eps) for i in range(1, K + 1)),
            W64 - sum(lr * g64 / (math.sqrt(1 - rho ** i) * np.abs(g64) + eps) for i in range(1, K + 1))]
    for got, w, name in zip(Ws, want, ("sgd", "momentum", "adagrad", "rmsprop")):
        ok, msg = close(got, w, 1e-5, 1e-6)
        assert ok, f"{name}: {msg}"
    assert close(st[0], -lr * g64 * (1 - mu ** K) / (1 - mu), 1e-5, 1e-9)[0]
    assert close(st[1], K * g64 * g64, 1e-5, 1e-12)[0]
    assert close(st[2], (1 - rho ** K) * g64 * g64, 1e-5, 1e-12)[0]
