"""Pins the oracle's Conv2D / MaxPool2D / Flatten (config 3) on the CPU:
reference known answers (tests/golden/known_answers.json) and float64 torch
conv2d / max_pool2d with autograd on NCHW tensors, which index
independently of the oracle's ColMajor arithmetic."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import ip
from oracle_lib import close, fp

GOLD = json.loads((Path(__file__).parent / "golden" / "known_answers.json").read_text())["cases"]


def to_cm(a: np.ndarray) -> np.ndarray:
    """Logical NCHW (any rank) -> flat Eigen ColMajor float32."""
    return np.ascontiguousarray(np.asarray(a, np.float32).transpose(*reversed(range(a.ndim)))).ravel()


def from_cm(flat, shape):
    return np.asarray(flat).reshape(tuple(reversed(shape))).transpose(*reversed(range(len(shape))))


@pytest.mark.parametrize("N,C,H,W,OC,KS,S,P", [(2, 3, 8, 8, 4, 3, 1, 1), (3, 2, 7, 5, 5, 3, 2, 0),
                                              (1, 4, 6, 6, 2, 2, 2, 1), (4, 3, 5, 5, 3, 1, 1, 0),
                                              (2, 5, 9, 7, 6, 5, 1, 2)])
def test_conv2d_vs_torch(oracle, N, C, H, W, OC, KS, S, P):
    rng = np.random.default_rng(N * 100 + C * 10 + KS)
    x = rng.standard_normal((N, C, H, W))
    w = rng.standard_normal((OC, C, KS, KS)) * 0.3
    b = rng.standard_normal(OC)
    HO, WO = (H + 2 * P - KS) // S + 1, (W + 2 * P - KS) // S + 1
    dy = rng.standard_normal((N, OC, HO, WO))
    X, Wt, B = to_cm(x), to_cm(w), b.astype(np.float32)
    Y = np.zeros(N * OC * HO * WO, np.float32)
    oracle.cnref_conv2d_forward(fp(X), fp(Wt), fp(B), fp(Y), N, C, H, W, OC, KS, S, P)
    gW, gb, dX = np.zeros_like(Wt), np.zeros(OC, np.float32), np.zeros_like(X)
    gW[:] = 7.0  # overwritten, not accumulated (conv2d.cpp:149-152)
    oracle.cnref_conv2d_backward(fp(X), fp(Wt), fp(to_cm(dy)), fp(gW), fp(gb), fp(dX), N, C, H, W,
                                 OC, KS, S, P)
    xt = torch.tensor(X.reshape(W, H, C, N).transpose(3, 2, 1, 0).astype(np.float64), requires_grad=True)
    wt = torch.tensor(Wt.reshape(KS, KS, C, OC).transpose(3, 2, 1, 0).astype(np.float64), requires_grad=True)
    bt = torch.tensor(B.astype(np.float64), requires_grad=True)
    yt = torch.nn.functional.conv2d(xt, wt, bt, stride=S, padding=P)
    yt.backward(torch.tensor(dy))
    for got, want, name in [(from_cm(Y, (N, OC, HO, WO)), yt.detach().numpy(), "Y"),
                            (from_cm(gW, (OC, C, KS, KS)), wt.grad.numpy(), "gW"),
                            (gb, bt.grad.numpy(), "gb"),
                            (from_cm(dX, (N, C, H, W)), xt.grad.numpy(), "dX")]:
        ok, msg = close(got, want, rtol=1e-5, atol=1e-5)
        assert ok, f"{name}: {msg}"


def test_conv2d_no_bias(oracle):
    N, C, H, W, OC, KS = 2, 2, 4, 4, 3, 3
    X = np.ones(N * C * H * W, np.float32)
    Wt = np.ones(OC * C * KS * KS, np.float32)
    Y = np.zeros(N * OC * 4 * 4, np.float32)
    oracle.cnref_conv2d_forward(fp(X), fp(Wt), None, fp(Y), N, C, H, W, OC, KS, 1, 1)
    y = from_cm(Y, (N, OC, 4, 4))
    # interior pixels see the full 3x3 window over 2 channels, corners a 2x2 window
    assert y[0, 0, 1, 1] == 18.0 and y[0, 0, 0, 0] == 8.0 and y[1, 2, 3, 0] == 8.0


def _pool_cases():
    return [c for c in GOLD if c["op"] == "maxpool2d_forward"]


@pytest.mark.parametrize("case", _pool_cases(), ids=lambda c: c["source"])
def test_maxpool_known_answers(oracle, case):
    x = np.asarray(case["X"], np.float32)
    N, C, H, W = x.shape
    p, s = case["pool"], case["stride"]
    HO, WO = (H - p) // s + 1, (W - p) // s + 1
    Y = np.zeros(N * C * HO * WO, np.float32)
    I = np.zeros(N * C * HO * WO, np.int32)
    oracle.cnref_maxpool2d_forward(fp(to_cm(x)), fp(Y), ip(I), N, C, H, W, p, s)
    np.testing.assert_allclose(from_cm(Y, (N, C, HO, WO)), case["expected"], atol=case["tol"])
    np.testing.assert_array_equal(from_cm(I, (N, C, HO, WO)), case["exact_argmax"])


@pytest.mark.parametrize("N,C,H,W,p,s", [(2, 3, 8, 8, 2, 2), (3, 2, 5, 5, 3, 1), (1, 4, 7, 9, 2, 3),
                                        (4, 2, 6, 6, 3, 2)])
def test_maxpool_vs_torch(oracle, N, C, H, W, p, s):
    rng = np.random.default_rng(N + C + H + W + p + s)
    x = rng.permutation(N * C * H * W).reshape(N, C, H, W).astype(np.float32)  # unique values
    HO, WO = (H - p) // s + 1, (W - p) // s + 1
    dy = rng.standard_normal((N, C, HO, WO)).astype(np.float32)
    Y = np.zeros(N * C * HO * WO, np.float32)
    I = np.zeros(N * C * HO * WO, np.int32)
    X = to_cm(x)
    oracle.cnref_maxpool2d_forward(fp(X), fp(Y), ip(I), N, C, H, W, p, s)
    dX = np.empty_like(X)
    oracle.cnref_maxpool2d_backward(fp(to_cm(dy)), ip(I), fp(dX), N, C, H, W, p, s)
    xt = torch.tensor(x.astype(np.float64), requires_grad=True)
    yt, it = torch.nn.functional.max_pool2d(xt, p, s, return_indices=True)
    yt.backward(torch.tensor(dy.astype(np.float64)))
    np.testing.assert_array_equal(from_cm(Y, (N, C, HO, WO)), yt.detach().numpy())
    # torch's index is flat h*W + w in the input plane; convert to window-local ph*p + pw
    ih, iw = it.numpy() // W, it.numpy() % W
    oh = np.arange(HO)[None, None, :, None]
    ow = np.arange(WO)[None, None, None, :]
    local = (ih - oh * s) * p + (iw - ow * s)
    np.testing.assert_array_equal(from_cm(I, (N, C, HO, WO)), local)
    ok, msg = close(from_cm(dX, (N, C, H, W)), xt.grad.numpy(), rtol=1e-6, atol=1e-7)
    assert ok, msg


def test_maxpool_ties_first_wins_and_minus_inf(oracle):
    x = np.zeros((1, 1, 2, 4), np.float32)
    x[0, 0] = [[1.0, 3.0, -np.inf, -np.inf], [3.0, 3.0, -np.inf, -np.inf]]
    Y, I = np.zeros(2, np.float32), np.zeros(2, np.int32)
    oracle.cnref_maxpool2d_forward(fp(to_cm(x)), fp(Y), ip(I), 1, 1, 2, 4, 2, 2)
    assert list(I) == [1, 0]  # first 3.0 at (0,1); all -inf -> index 0 (never >)
    assert Y[0] == 3.0 and Y[1] == -np.inf


def test_flatten_is_colmajor_reshape():
    (case,) = [c for c in GOLD if c["op"] == "flatten_forward"]
    x = np.asarray(case["X"], np.float32)
    flat = to_cm(x)  # the same buffer viewed as [N, C*H*W] ColMajor
    out = from_cm(flat, case["expected_shape"])
    np.testing.assert_array_equal(out, case["exact"])
    assert out.sum() == x.sum() == 36.0
