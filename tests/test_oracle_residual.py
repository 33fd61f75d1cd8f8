"""Pins the Residual restatement (oracle cnref_residual_*, residual.cpp:23-159)
and the residual-network composition (oracle/resnet.py) on the CPU:

* known answers: the reference's own skip-connection test
  (tests/layers/test_residual.cpp:68-84) and two hand-derived cases, one with
  the projection shortcut (tests/golden/known_answers.json);
* float64 torch autograd of block(x) + shortcut(x) for a two-Linear block,
  with and without the projection, including the Linear layers' gradient
  accumulation across two backward calls (linear.cpp:346-352);
* one train step of the residual benchmark network (identity shortcuts, and
  a last block with a projection) against float64 autograd: loss, every
  gradient, and the step-1 Adam update.
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from cppnet_amd import trainer
from oracle.resnet import OracleResNet, residual_backward, residual_forward, resnet_layout
from oracle_lib import colmajor, from_colmajor
from test_oracle_models import _check, from_cm, t64

GOLD = json.loads((Path(__file__).parent / "golden" / "known_answers.json").read_text())["cases"]


def _cases(op):
    return [c for c in GOLD if c["op"] == op]


def _block(case):
    Ws, bs, sizes = [], [], None
    for layer in case["block"]:
        W = np.asarray(layer["W"], np.float32)
        sizes = [W.shape[0]] if sizes is None else sizes
        sizes.append(W.shape[1])
        Ws.append(colmajor(W))
        bs.append(None if layer["b"] is None else np.asarray(layer["b"], np.float32))
    Wp = None if case["Wp"] is None else colmajor(np.asarray(case["Wp"], np.float32))
    return Ws, bs, Wp, sizes


@pytest.mark.parametrize("case", _cases("residual_forward"), ids=lambda c: c["source"])
def test_known_residual_forward(oracle, case):
    Ws, bs, Wp, sizes = _block(case)
    X = np.asarray(case["X"], np.float32)
    B = X.shape[0]
    y, _ = residual_forward(oracle, Ws, bs, Wp, colmajor(X), B, sizes)
    got = from_colmajor(y, B, sizes[-1])
    np.testing.assert_allclose(got, case["exact"], rtol=0, atol=case["tol"])
    if "expected" in case:
        np.testing.assert_allclose(got, case["expected"], rtol=0, atol=case["tol"])


@pytest.mark.parametrize("case", _cases("residual_backward"), ids=lambda c: c["source"])
def test_known_residual_backward(oracle, case):
    Ws, bs, Wp, sizes = _block(case)
    X = np.asarray(case["X"], np.float32)
    B = X.shape[0]
    x = colmajor(X)
    _, acts = residual_forward(oracle, Ws, bs, Wp, x, B, sizes)
    gW = [np.zeros_like(w) for w in Ws]
    gb = [None if b is None else np.zeros_like(b) for b in bs]
    dX = residual_backward(oracle, Ws, Wp, x, acts, colmajor(np.asarray(case["dY"], np.float32)), gW, gb, None,
                           B, sizes)
    np.testing.assert_allclose(from_colmajor(dX, B, sizes[0]), case["exact"], atol=case["tol"])
    for k, want in enumerate(case["exact_gW"]):
        np.testing.assert_allclose(from_colmajor(gW[k], sizes[k], sizes[k + 1]), want, atol=case["tol"])
    for k, want in enumerate(case["exact_gb"]):
        np.testing.assert_allclose(gb[k], want, atol=case["tol"])


@pytest.mark.parametrize("proj", [False, True])
def test_residual_vs_autograd_with_accumulation(oracle, proj):
    rng = np.random.default_rng(5)
    B, I, H = 5, 6, 9
    O = 4 if proj else I
    sizes = [I, H, O]
    Wl = [rng.standard_normal((I, H)), rng.standard_normal((H, O))]
    bl = [rng.standard_normal(H), rng.standard_normal(O)]
    Wp = rng.standard_normal((I, O)) if proj else None
    X = rng.standard_normal((B, I))
    dYs = [rng.standard_normal((B, O)) for _ in range(2)]
    # oracle: two forward/backward passes; grads accumulate across them
    Ws = [colmajor(w.astype(np.float32)) for w in Wl]
    bs = [b.astype(np.float32) for b in bl]
    Wpc = colmajor(Wp.astype(np.float32)) if proj else None
    gW = [np.zeros_like(w) for w in Ws]
    gb = [np.zeros_like(b) for b in bs]
    gWp = np.zeros_like(Wpc) if proj else None
    x = colmajor(X.astype(np.float32))
    for dY in dYs:
        y, acts = residual_forward(oracle, Ws, bs, Wpc, x, B, sizes)
        dX = residual_backward(oracle, Ws, Wpc, x, acts, colmajor(dY.astype(np.float32)), gW, gb, gWp, B, sizes)
    # float64 autograd, same two passes
    Wt = [torch.tensor(w, requires_grad=True) for w in Wl]
    bt = [torch.tensor(b, requires_grad=True) for b in bl]
    Wpt = torch.tensor(Wp, requires_grad=True) if proj else None
    for dY in dYs:
        xt = torch.tensor(X, requires_grad=True)
        yt = (xt @ Wt[0] + bt[0]) @ Wt[1] + bt[1] + (xt @ Wpt if proj else xt)
        yt.backward(torch.tensor(dY))
    np.testing.assert_allclose(from_colmajor(y, B, O), yt.detach().numpy(), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(from_colmajor(dX, B, I), xt.grad.numpy(), rtol=1e-5, atol=1e-5)
    for k in range(2):
        np.testing.assert_allclose(from_colmajor(gW[k], sizes[k], sizes[k + 1]), Wt[k].grad.numpy(), rtol=1e-5,
                                   atol=1e-5)
        np.testing.assert_allclose(gb[k], bt[k].grad.numpy(), rtol=1e-5, atol=1e-5)
    if proj:
        np.testing.assert_allclose(from_colmajor(gWp, I, O), Wpt.grad.numpy(), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("last_width", [0, 12])
def test_resnet_step_vs_autograd(oracle, last_width):
    cfg = trainer.ResNetConfig("small resnet", 5, 16, 2, 4, 10, last_width=last_width)
    params, X, Y = trainer.synthetic_resnet(cfg, np.random.default_rng(6))
    ref = OracleResNet(cfg, oracle)
    ref.set_params(params)
    loss = ref.step(X, Y)
    shapes, blocks = resnet_layout(cfg)
    assert [int(np.prod(s)) for s in shapes] == [p.size for p in params]
    P = [t64(from_cm(p, s)) for p, s in zip(params, shapes)]
    B = cfg.batch
    h = torch.relu(torch.tensor(from_cm(X, (B, cfg.in_features)), dtype=torch.float64) @ P[0] + P[1])
    k = 2
    for (w_in, W, w_out) in blocks:
        f = (h @ P[k] + P[k + 1]) @ P[k + 2] + P[k + 3]
        if w_out != w_in:
            h = torch.relu(f + h @ P[k + 4])
            k += 5
        else:
            h = torch.relu(f + h)
            k += 4
    z = h @ P[k] + P[k + 1]
    t = torch.tensor(from_cm(Y, (B, cfg.classes)), dtype=torch.float64)
    lt = -(t * torch.log_softmax(z, 1)).sum() / B
    lt.backward()
    _check(ref, loss, lt, params, P, shapes, cfg.lr, cfg.eps)
