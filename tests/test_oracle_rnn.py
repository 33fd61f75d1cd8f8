"""Pins the oracle's LSTM and GRU (CPU only).

* Closed forms: with zero weights the recurrences are geometric series:
  LSTM c_t = i g (1 - f^t)/(1 - f), h_t = o tanh(c_t) with i, f, g, o fixed by
  the biases; GRU h_t = n (1 - z^t).  These pin the forward recurrence, the
  gate order (i,f,g,o / z,r,n) and the forget-gate convention.
* Gradients: float64 torch autograd through the same forward equations
  (lstm.cpp:104-134, gru.cpp:102-135) on logical [B, S, I] tensors; the hand
  derived BPTT of the oracle must match automatic differentiation.
"""
import numpy as np
import pytest
import torch

from oracle_lib import close, fp


def cm(a):
    a = np.asarray(a, np.float32)
    return np.ascontiguousarray(a.transpose(*reversed(range(a.ndim)))).ravel()


def from_cm(flat, shape):
    return np.asarray(flat).reshape(tuple(reversed(shape))).transpose(*reversed(range(len(shape))))


def run_lstm(oracle, x, Wih, Whh, b):
    B, S, I = x.shape
    H = Whh.shape[0]
    Y = np.zeros(B * S * H, np.float32)
    gates = np.zeros(B * S * 4 * H, np.float32)
    c, tc = np.zeros(B * S * H, np.float32), np.zeros(B * S * H, np.float32)
    X = cm(x)
    oracle.cnref_lstm_forward(fp(X), fp(cm(Wih)), fp(cm(Whh)), fp(b.astype(np.float32)), fp(Y),
                              fp(gates), fp(c), fp(tc), B, S, I, H)
    return X, Y, gates, c, tc


def test_lstm_zero_weight_closed_form(oracle):
    B, S, I, H = 3, 6, 4, 5
    rng = np.random.default_rng(0)
    b = rng.standard_normal(4 * H).astype(np.float32)
    x = rng.standard_normal((B, S, I))
    _, Y, _, c, _ = run_lstm(oracle, x, np.zeros((I, 4 * H)), np.zeros((H, 4 * H)), b)
    sig = lambda v: 1 / (1 + np.exp(-v.astype(np.float64)))
    i, f, g, o = sig(b[:H]), sig(b[H:2 * H]), np.tanh(b[2 * H:3 * H].astype(np.float64)), sig(b[3 * H:])
    y = from_cm(Y, (B, S, H))
    for t in range(S):
        ct = i * g * (1 - f ** (t + 1)) / (1 - f)
        np.testing.assert_allclose(y[:, t, :], np.broadcast_to(o * np.tanh(ct), (B, H)), rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(from_cm(c, (B * S, H))[t * B:(t + 1) * B], np.broadcast_to(ct, (B, H)),
                                   rtol=1e-5, atol=1e-6)


def torch_lstm(x, Wih, Whh, b):
    B, S, _ = x.shape
    H = Whh.shape[0]
    h = torch.zeros(B, H, dtype=torch.float64)
    c = torch.zeros(B, H, dtype=torch.float64)
    out = []
    for t in range(S):
        gts = x[:, t, :] @ Wih + h @ Whh + b
        i, f = torch.sigmoid(gts[:, :H]), torch.sigmoid(gts[:, H:2 * H])
        g, o = torch.tanh(gts[:, 2 * H:3 * H]), torch.sigmoid(gts[:, 3 * H:])
        c = f * c + i * g
        h = o * torch.tanh(c)
        out.append(h)
    return torch.stack(out, 1)


@pytest.mark.parametrize("B,S,I,H", [(2, 5, 3, 4), (4, 3, 6, 8), (1, 1, 2, 3)])
def test_lstm_backward_vs_autograd(oracle, B, S, I, H):
    rng = np.random.default_rng(B * 10 + S)
    x = rng.standard_normal((B, S, I))
    Wih = rng.standard_normal((I, 4 * H)) * 0.4
    Whh = rng.standard_normal((H, 4 * H)) * 0.4
    b = rng.standard_normal(4 * H) * 0.5
    b[H:2 * H] += 1.0  # the constructor's forget bias (lstm.cpp:47-49)
    dy = rng.standard_normal((B, S, H))
    X, Y, gates, c, tc = run_lstm(oracle, x, Wih, Whh, b)
    gWih, gWhh = np.full(I * 4 * H, 9.0, np.float32), np.full(H * 4 * H, 9.0, np.float32)
    gb, dX = np.full(4 * H, 9.0, np.float32), np.zeros_like(X)
    oracle.cnref_lstm_backward(fp(X), fp(cm(Wih)), fp(cm(Whh)), fp(Y), fp(gates), fp(c), fp(tc),
                               fp(cm(dy)), fp(gWih), fp(gWhh), fp(gb), fp(dX), B, S, I, H)
    t = [torch.tensor(v, dtype=torch.float64, requires_grad=True) for v in (x, Wih, Whh, b)]
    yt = torch_lstm(*t)
    yt.backward(torch.tensor(dy))
    checks = [(from_cm(Y, (B, S, H)), yt.detach().numpy(), "Y"),
              (from_cm(gWih, (I, 4 * H)), t[1].grad.numpy(), "gW_ih"),
              (from_cm(gWhh, (H, 4 * H)), t[2].grad.numpy(), "gW_hh"),
              (gb, t[3].grad.numpy(), "gb"), (from_cm(dX, (B, S, I)), t[0].grad.numpy(), "dX")]
    for got, want, name in checks:
        ok, msg = close(got, want, rtol=2e-5, atol=2e-6)
        assert ok, f"{name}: {msg}"


def run_gru(oracle, x, Wih, Whh, b):
    B, S, I = x.shape
    H = Whh.shape[0]
    Y = np.zeros(B * S * H, np.float32)
    gates, rh = np.zeros(B * S * 3 * H, np.float32), np.zeros(B * S * H, np.float32)
    X = cm(x)
    oracle.cnref_gru_forward(fp(X), fp(cm(Wih)), fp(cm(Whh)), fp(b.astype(np.float32)), fp(Y),
                             fp(gates), fp(rh), B, S, I, H)
    return X, Y, gates, rh


def test_gru_zero_weight_closed_form(oracle):
    B, S, I, H = 2, 7, 3, 4
    rng = np.random.default_rng(1)
    b = rng.standard_normal(3 * H).astype(np.float32)
    _, Y, _, _ = run_gru(oracle, rng.standard_normal((B, S, I)), np.zeros((I, 3 * H)),
                         np.zeros((H, 3 * H)), b)
    z = 1 / (1 + np.exp(-b[:H].astype(np.float64)))
    n = np.tanh(b[2 * H:].astype(np.float64))
    y = from_cm(Y, (B, S, H))
    for t in range(S):
        np.testing.assert_allclose(y[:, t, :], np.broadcast_to(n * (1 - z ** (t + 1)), (B, H)),
                                   rtol=1e-5, atol=1e-6)


def torch_gru(x, Wih, Whh, b):
    B, S, _ = x.shape
    H = Whh.shape[0]
    h = torch.zeros(B, H, dtype=torch.float64)
    out = []
    for t in range(S):
        xg = x[:, t, :] @ Wih
        hg = h @ Whh
        z = torch.sigmoid(xg[:, :H] + hg[:, :H] + b[:H])
        r = torch.sigmoid(xg[:, H:2 * H] + hg[:, H:2 * H] + b[H:2 * H])
        n = torch.tanh(xg[:, 2 * H:] + (r * h) @ Whh[:, 2 * H:] + b[2 * H:])
        h = (1 - z) * n + z * h
        out.append(h)
    return torch.stack(out, 1)


@pytest.mark.parametrize("B,S,I,H", [(2, 5, 3, 4), (3, 4, 5, 6), (1, 1, 2, 2)])
def test_gru_backward_vs_autograd(oracle, B, S, I, H):
    rng = np.random.default_rng(B * 7 + S)
    x = rng.standard_normal((B, S, I))
    Wih = rng.standard_normal((I, 3 * H)) * 0.4
    Whh = rng.standard_normal((H, 3 * H)) * 0.4
    b = rng.standard_normal(3 * H) * 0.5
    dy = rng.standard_normal((B, S, H))
    X, Y, gates, rh = run_gru(oracle, x, Wih, Whh, b)
    gWih, gWhh = np.full(I * 3 * H, 9.0, np.float32), np.full(H * 3 * H, 9.0, np.float32)
    gb, dX = np.full(3 * H, 9.0, np.float32), np.zeros_like(X)
    oracle.cnref_gru_backward(fp(X), fp(cm(Wih)), fp(cm(Whh)), fp(Y), fp(gates), fp(rh), fp(cm(dy)),
                              fp(gWih), fp(gWhh), fp(gb), fp(dX), B, S, I, H)
    t = [torch.tensor(v, dtype=torch.float64, requires_grad=True) for v in (x, Wih, Whh, b)]
    yt = torch_gru(*t)
    yt.backward(torch.tensor(dy))
    checks = [(from_cm(Y, (B, S, H)), yt.detach().numpy(), "Y"),
              (from_cm(gWih, (I, 3 * H)), t[1].grad.numpy(), "gW_ih"),
              (from_cm(gWhh, (H, 3 * H)), t[2].grad.numpy(), "gW_hh"),
              (gb, t[3].grad.numpy(), "gb"), (from_cm(dX, (B, S, I)), t[0].grad.numpy(), "dX")]
    for got, want, name in checks:
        ok, msg = close(got, want, rtol=2e-5, atol=2e-6)
        assert ok, f"{name}: {msg}"
