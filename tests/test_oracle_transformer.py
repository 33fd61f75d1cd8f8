"""Pins the oracle's config-5 ops (CPU only): Embedding, MultiHeadAttention,
BatchNorm, GELU, MeanPool1D.  References: the reference tests' checks
(BN per-feature mean 0 / var 1, tests/layers/test_batch_norm.cpp:51-66;
lookup = weight row, tests/layers/test_embedding.cpp:50-60) and float64 torch
autograd on logical tensors (independent of the oracle's ColMajor loops)."""
import numpy as np
import pytest
import torch

from oracle import ip
from oracle_lib import close, fp


def cm(a):
    a = np.asarray(a, np.float32)
    return np.ascontiguousarray(a.transpose(*reversed(range(a.ndim)))).ravel()


def from_cm(flat, shape):
    return np.asarray(flat).reshape(tuple(reversed(shape))).transpose(*reversed(range(len(shape))))


def t64(a):
    return torch.tensor(np.asarray(a, np.float64), requires_grad=True)


def test_embedding_lookup_scatter_and_bounds(oracle):
    B, S, V, D = 3, 5, 7, 4
    rng = np.random.default_rng(0)
    ids = rng.integers(0, V, (B, S)).astype(np.int32)
    ids[0, :3] = 2  # duplicate ids accumulate
    W = rng.standard_normal((V, D)).astype(np.float32)
    out = np.zeros(B * S * D, np.float32)
    assert oracle.cnref_embedding_forward(ip(cm(ids).astype(np.int32)), fp(cm(W)), fp(out), B, S, V, D) == 0
    np.testing.assert_array_equal(from_cm(out, (B, S, D)), W[ids])  # exact row routing
    dY = rng.standard_normal((B, S, D)).astype(np.float32)
    gW = np.full(V * D, 5.0, np.float32)
    oracle.cnref_embedding_backward(ip(cm(ids).astype(np.int32)), fp(cm(dY)), fp(gW), B, S, V, D)
    Wt = t64(W)
    torch.nn.functional.embedding(torch.tensor(ids, dtype=torch.long), Wt).backward(torch.tensor(dY, dtype=torch.float64))
    ok, msg = close(from_cm(gW, (V, D)), Wt.grad.numpy(), 1e-6, 1e-7)
    assert ok, msg
    untouched = np.setdiff1d(np.arange(V), ids.ravel())
    assert not from_cm(gW, (V, D))[untouched].any()  # rows never looked up stay exactly 0
    bad = cm(ids).astype(np.int32)
    bad[4] = V
    assert oracle.cnref_embedding_forward(ip(bad), fp(cm(W)), fp(out), B, S, V, D) == -1


def torch_mha(q, k, v, Wq, Wk, Wv, Wo, heads):
    D = Wq.shape[0]
    scale = 1.0 / np.sqrt(np.float32(D // heads))
    Qp, Kp, Vp = q @ Wq, k @ Wk, v @ Wv            # [B, S, D]
    A = torch.softmax((Qp @ Kp.transpose(1, 2).contiguous()) * scale, dim=-1)
    return (A @ Vp) @ Wo, A


@pytest.mark.parametrize("B,S,D,h", [(2, 5, 8, 2), (3, 7, 12, 4), (1, 1, 4, 1)])
def test_mha_vs_autograd(oracle, B, S, D, h):
    rng = np.random.default_rng(B + S + D)
    x = rng.standard_normal((B, S, D))
    Ws = [rng.standard_normal((D, D)) * 0.3 for _ in range(4)]
    dy = rng.standard_normal((B, S, D))
    X = cm(x)
    out, attn = np.zeros(B * S * D, np.float32), np.zeros(B * S * S, np.float32)
    Wc = [cm(w) for w in Ws]
    oracle.cnref_mha_forward(fp(X), fp(X), fp(X), *[fp(w) for w in Wc], fp(out), fp(attn), B, S, D, h)
    g = [np.full(D * D, 3.0, np.float32) for _ in range(4)]
    dX = np.zeros_like(X)
    oracle.cnref_mha_backward(fp(X), fp(X), fp(X), *[fp(w) for w in Wc], fp(attn), fp(cm(dy)),
                              *[fp(a) for a in g], fp(dX), B, S, D, h)
    xt = t64(x)
    wt = [t64(w) for w in Ws]
    yt, At = torch_mha(xt, xt, xt, *wt, h)
    yt.backward(torch.tensor(dy))
    checks = [(from_cm(out, (B, S, D)), yt.detach().numpy(), "out"),
              (from_cm(attn, (B, S, S)), At.detach().numpy(), "attn"),
              (from_cm(dX, (B, S, D)), xt.grad.numpy(), "dX")]
    checks += [(from_cm(a, (D, D)), w.grad.numpy(), f"gW{n}") for a, w, n in zip(g, wt, "qkvo")]
    for got, want, name in checks:
        ok, msg = close(got, want, 2e-5, 2e-6)
        assert ok, f"{name}: {msg}"


def test_batchnorm_known_properties_and_autograd(oracle):
    N, F = 64, 6
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((N, F)) * 3 + 2).astype(np.float32)
    gamma = (1 + 0.3 * rng.standard_normal(F)).astype(np.float32)
    beta = rng.standard_normal(F).astype(np.float32)
    rm, rv = np.zeros(F, np.float32), np.ones(F, np.float32)
    bm, bv = np.zeros(F, np.float32), np.zeros(F, np.float32)
    y, xh = np.zeros(N * F, np.float32), np.zeros(N * F, np.float32)
    oracle.cnref_batchnorm_forward(fp(cm(x)), fp(y), fp(xh), fp(gamma), fp(beta), fp(rm), fp(rv),
                                   fp(bm), fp(bv), N, F, 0.1, 1e-5)
    xhat = from_cm(xh, (N, F))
    np.testing.assert_allclose(xhat.mean(0), 0, atol=1e-5)  # test_batch_norm.cpp:51-66
    np.testing.assert_allclose(xhat.var(0), 1, atol=1e-3)
    np.testing.assert_allclose(rm, 0.1 * x.mean(0, dtype=np.float64), rtol=1e-5)
    np.testing.assert_allclose(rv, 0.9 + 0.1 * x.var(0, dtype=np.float64), rtol=1e-5)  # biased var
    dy = rng.standard_normal((N, F)).astype(np.float32)
    gg, gbt, dX = np.zeros(F, np.float32), np.zeros(F, np.float32), np.zeros(N * F, np.float32)
    oracle.cnref_batchnorm_backward(fp(cm(dy)), fp(cm(x)), fp(xh), fp(gamma), fp(bm), fp(bv), fp(gg),
                                    fp(gbt), fp(dX), N, F, 1e-5)
    xt, gt, bt = t64(x), t64(gamma), t64(beta)
    yt = torch.nn.functional.batch_norm(xt, None, None, gt, bt, training=True, eps=1e-5)
    yt.backward(torch.tensor(dy, dtype=torch.float64))
    for got, want, name in [(from_cm(y, (N, F)), yt.detach().numpy(), "y"),
                            (from_cm(dX, (N, F)), xt.grad.numpy(), "dX"),
                            (gg, gt.grad.numpy(), "ggamma"), (gbt, bt.grad.numpy(), "gbeta")]:
        ok, msg = close(got, want, 1e-4, 1e-5)
        assert ok, f"{name}: {msg}"


def test_gelu_vs_autograd(oracle):
    x = np.linspace(-6, 6, 1001).astype(np.float32)
    dy = np.cos(x).astype(np.float32)
    y, dx = np.zeros_like(x), np.zeros_like(x)
    oracle.cnref_gelu_forward(fp(x), fp(y), x.size)
    oracle.cnref_gelu_backward(fp(x), fp(dy), fp(dx), x.size)
    xt = t64(x)
    yt = torch.nn.functional.gelu(xt)
    yt.backward(torch.tensor(dy, dtype=torch.float64))
    ok, msg = close(y, yt.detach().numpy(), 1e-6, 1e-7)
    assert ok, msg
    ok, msg = close(dx, xt.grad.numpy(), 1e-6, 1e-7)
    assert ok, msg
    assert y[500] == 0.0 and abs(dx[500] - 0.5 * dy[500]) < 1e-7  # GELU(0) = 0, GELU'(0) = 1/2


def test_meanpool1d_vs_autograd(oracle):
    B, S, D = 3, 7, 5
    rng = np.random.default_rng(4)
    x, dy = rng.standard_normal((B, S, D)), rng.standard_normal((B, D))
    y, dx = np.zeros(B * D, np.float32), np.zeros(B * S * D, np.float32)
    oracle.cnref_meanpool1d_forward(fp(cm(x)), fp(y), B, S, D)
    oracle.cnref_meanpool1d_backward(fp(cm(dy)), fp(dx), B, S, D)
    xt = t64(x)
    yt = xt.mean(1)
    yt.backward(torch.tensor(dy))
    ok, msg = close(from_cm(y, (B, D)), yt.detach().numpy(), 1e-6, 1e-7)
    assert ok, msg
    ok, msg = close(from_cm(dx, (B, S, D)), xt.grad.numpy(), 1e-6, 1e-7)
    assert ok, msg


def test_transformer_train_step_vs_autograd(oracle):
    """The config-5 composition of the oracle (oracle/transformer.py) against
    float64 torch autograd of the same network on logical tensors: loss, every
    parameter gradient and the Adam-updated parameters."""
    from cppnet_amd import trainer
    from oracle.transformer import OracleTransformer
    cfg = trainer.transformer_config(5, batch=3, seq_len=5, vocab=13, embed_dim=8, heads=2, blocks=2,
                                     ffn=12, classes=3)
    params, ids, Y = trainer.synthetic_transformer(cfg, np.random.default_rng(9))
    ref = OracleTransformer(cfg, oracle)
    ref.set_params(params)
    loss = ref.step(ids, Y)
    B, S, V, D, F, C = cfg.batch, cfg.seq_len, cfg.vocab, cfg.embed_dim, cfg.ffn, cfg.classes
    shapes = [(V, D)] + [(D, D)] * 4 + [(D,), (D,), (D, F), (F,), (F, D), (D,)]
    shapes = shapes[:1] + shapes[1:] * cfg.blocks + [(D, C), (C,)]
    P = [t64(from_cm(p, s)) for p, s in zip(params, shapes)]
    tok = torch.tensor(from_cm(ids, (B, S)), dtype=torch.long)
    x = P[0][tok]
    for i in range(cfg.blocks):
        Wq, Wk, Wv, Wo, g, b, W1, b1, W2, b2 = P[1 + 10 * i: 11 + 10 * i]
        a, _ = torch_mha(x, x, x, Wq, Wk, Wv, Wo, cfg.heads)
        r = (a + x).reshape(B * S, D)
        h = torch.nn.functional.batch_norm(r, None, None, g, b, training=True, eps=1e-5)
        y = torch.nn.functional.gelu(h @ W1 + b1) @ W2 + b2 + h
        x = y.reshape(B, S, D)
    logits = x.mean(1) @ P[-2] + P[-1]
    t = torch.tensor(from_cm(Y, (B, C)), dtype=torch.float64)
    lt = -(t * torch.log_softmax(logits, 1)).sum() / B
    lt.backward()
    assert abs(loss - lt.item()) <= 1e-5 * abs(lt.item())
    for k, (gr, p, s) in enumerate(zip(ref.last_grads, P, shapes)):
        want = p.grad.numpy()
        scale = np.abs(want).max() + 1e-30
        err = np.abs(from_cm(gr, s) - want).max() / scale
        assert err < 1e-4, f"grad of param {k}: max err {err:.3g} of max |g| {scale:.3g}"
    # Adam step 1: W - lr * g / (|g| + eps) exactly in the limit (closed form)
    for k, (p_new, p0, gr) in enumerate(zip(ref.get_params(), params, ref.last_grads)):
        g64 = gr.astype(np.float64)
        want = p0 - cfg.lr * g64 / (np.abs(g64) + cfg.eps)
        np.testing.assert_allclose(p_new, want, rtol=1e-6, atol=1e-8, err_msg=f"param {k}")
