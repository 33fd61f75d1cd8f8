"""Pins the oracle's model compositions (oracle/mlp.py, oracle/cnn.py,
oracle/rnn.py; oracle/transformer.py is pinned in test_oracle_transformer.py)
on the CPU: one train step of each benchmark network at a small shape
against float64 torch autograd of the same network on logical tensors --
the loss, every parameter gradient, and the Adam-updated parameters (step 1
closed form W - lr g / (|g| + eps)).  A wiring mistake in a composition (a
layer order, a transposed operand, a missing bias) fails one of these."""
import numpy as np
import pytest
import torch

from cppnet_amd import trainer
from test_oracle_rnn import torch_gru, torch_lstm


def from_cm(flat, shape):
    return np.asarray(flat).reshape(tuple(reversed(shape))).transpose(*reversed(range(len(shape))))


def t64(a):
    return torch.tensor(np.asarray(a, np.float64), requires_grad=True)


def _check(ref, loss, lt, params, P, shapes, lr, eps):
    assert abs(loss - lt.item()) <= 1e-5 * abs(lt.item()) + 1e-7, (loss, lt.item())
    for k, (gr, p, s) in enumerate(zip(ref.last_grads, P, shapes)):
        want = p.grad.numpy()
        scale = np.abs(want).max() + 1e-30
        err = np.abs(from_cm(gr, s) - want).max() / scale
        assert err < 1e-4, f"grad of param {k}: max err {err:.3g} of max |g| {scale:.3g}"
    for k, (p_new, p0, gr) in enumerate(zip(ref.get_params(), params, ref.last_grads)):
        g64 = gr.astype(np.float64)
        np.testing.assert_allclose(p_new, p0 - lr * g64 / (np.abs(g64) + eps), rtol=1e-6, atol=1e-8,
                                   err_msg=f"param {k}")


@pytest.mark.parametrize("kind", ["c1", "c2"])
def test_mlp_step_vs_autograd(oracle, kind):
    from oracle.mlp import OracleMLP
    if kind == "c1":
        cfg = trainer.mlp_config(1, batch=16)
    else:
        cfg = trainer.mlp_config(2, batch=12)
        cfg.sizes = [16, 32, 24, 10]
    params, X, Y = trainer.synthetic_mlp(cfg, np.random.default_rng(3))
    ref = OracleMLP(cfg, oracle)
    ref.set_params(params)
    loss = ref.step(X, Y)
    B, sz = cfg.batch, cfg.sizes
    shapes = [s for i, o in zip(sz[:-1], sz[1:]) for s in ((i, o), (o,))]
    P = [t64(from_cm(p, s)) for p, s in zip(params, shapes)]
    h = torch.tensor(from_cm(X, (B, sz[0])), dtype=torch.float64)
    n = len(sz) - 1
    for i in range(n):
        h = h @ P[2 * i] + P[2 * i + 1]
        if i + 1 < n:
            h = torch.relu(h)
    t = torch.tensor(from_cm(Y, (B, sz[-1])), dtype=torch.float64)
    if cfg.loss == "bce":
        p = torch.sigmoid(h).clamp(1e-7, 1 - 1e-7)
        lt = -(t * torch.log(p) + (1 - t) * torch.log(1 - p)).mean()
    else:
        lt = -(t * torch.log_softmax(h, 1)).sum() / B
    lt.backward()
    _check(ref, loss, lt, params, P, shapes, cfg.lr, cfg.eps)


def test_cnn_step_vs_autograd(oracle):
    from oracle.cnn import OracleCNN
    cfg = trainer.CNNConfig("small CNN", [(3, 4, 3, 1, 1), (4, 6, 3, 1, 1)], 2, [4, 3, 8, 8], 5)
    params, X, Y = trainer.synthetic_cnn(cfg, np.random.default_rng(4))
    ref = OracleCNN(cfg, oracle)
    ref.set_params(params)
    loss = ref.step(X, Y)
    N = cfg.batch
    shapes = []
    for (ic, oc, k, _, _) in cfg.convs:
        shapes += [(oc, ic, k, k), (oc,)]
    F = cfg.flat_features()
    shapes += [(F, cfg.classes), (cfg.classes,)]
    P = [t64(from_cm(p, s)) for p, s in zip(params, shapes)]
    h = torch.tensor(from_cm(X, tuple(cfg.input_shape)), dtype=torch.float64)
    for i, (_, _, _, s, pd) in enumerate(cfg.convs):
        h = torch.nn.functional.conv2d(h, P[2 * i], P[2 * i + 1], stride=s, padding=pd)
        h = torch.nn.functional.max_pool2d(torch.relu(h), cfg.pool)
    # Flatten is the ColMajor reshape: feature index c + C*(h + H*w)
    h = h.permute(0, 3, 2, 1).reshape(N, -1)
    logits = h @ P[-2] + P[-1]
    t = torch.tensor(from_cm(Y, (N, cfg.classes)), dtype=torch.float64)
    lt = -(t * torch.log_softmax(logits, 1)).sum() / N
    lt.backward()
    _check(ref, loss, lt, params, P, shapes, cfg.lr, cfg.eps)


@pytest.mark.parametrize("cell", ["lstm", "gru"])
def test_seq_regressor_step_vs_autograd(oracle, cell):
    from oracle.rnn import OracleSeqRegressor
    cfg = trainer.rnn_config(4, batch=3, seq_len=5, cell=cell)
    cfg.input_size, cfg.hidden = 4, 6
    params, X, Y = trainer.synthetic_rnn(cfg, np.random.default_rng(5))
    ref = OracleSeqRegressor(cfg, oracle)
    ref.set_params(params)
    loss = ref.step(X, Y)
    B, S, I, H, O = cfg.batch, cfg.seq_len, cfg.input_size, cfg.hidden, cfg.out_features
    G = (4 if cell == "lstm" else 3) * H
    shapes = [(I, G), (H, G), (G,), (H, O), (O,)]
    P = [t64(from_cm(p, s)) for p, s in zip(params, shapes)]
    x = torch.tensor(from_cm(X, (B, S, I)), dtype=torch.float64)
    seq = (torch_lstm if cell == "lstm" else torch_gru)(x, P[0], P[1], P[2])
    pred = seq[:, S - 1, :] @ P[3] + P[4]
    t = torch.tensor(from_cm(Y, (B, O)), dtype=torch.float64)
    lt = ((pred - t) ** 2).mean()
    lt.backward()
    _check(ref, loss, lt, params, P, shapes, cfg.lr, cfg.eps)
