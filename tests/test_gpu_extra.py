"""GPU parity of the reference's device ops off the BASELINE configs against
the CPU oracle (oracle/cnref_extra.cpp).

Bit-exact where the kernel evaluates the reference's operations in the
reference's order with one rounding each: LeakyReLU, the MAE / Huber / CCE
gradients, the four optimizer updates, Dropout given its mask (and the mask
itself against an independent restatement of its generator), both global
pools (sums in the reference's h-then-w order; the max scan and its argmax).
Within rel 1e-5 where a transcendental is involved (softmax, the CCE loss,
whose exp/log differ from the host's by an ulp); losses reduced in a
different order within rel 2e-4 of their size (the oracle's
sequential fp32 sum of up to 2^18 terms carries ~u*sqrt(n) itself); the RNN within rel 1e-4 /
abs 1e-5 with magnitude-aware contractions, as the LSTM tests.
"""
import numpy as np
import pytest
import torch

from cppnet_amd import ops
from oracle_lib import close, close_mag, fp, gemm_mag

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def ip(a):
    import ctypes as C
    return a.ctypes.data_as(C.POINTER(C.c_int32))


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def _edges(rng, n):
    x = rng.standard_normal(n).astype(np.float32) * 3
    x[:6] = [0.0, -0.0, 1e-30, -1e-30, 1e30, -1e30]
    return x


@pytest.mark.parametrize("n", [1, 7, 4096, 1 << 20])
def test_leaky_relu_exact(gpu, oracle, n):
    rng = np.random.default_rng(n)
    x, dy = _edges(rng, max(n, 6))[:n], rng.standard_normal(n).astype(np.float32)
    for alpha in (0.01, 0.2, 0.0):
        y, dx = torch.empty(n, device="cuda"), torch.empty(n, device="cuda")
        ops.leaky_relu_forward(dev(x), y, alpha)
        ops.leaky_relu_backward(dev(x), dev(dy), dx, alpha)
        ry, rdx = np.zeros(n, np.float32), np.zeros(n, np.float32)
        oracle.cnref_leaky_relu_forward(fp(x), fp(ry), n, alpha)
        oracle.cnref_leaky_relu_backward(fp(x), fp(dy), fp(rdx), n, alpha)
        np.testing.assert_array_equal(bits(host(y)), bits(ry))
        np.testing.assert_array_equal(bits(host(dx)), bits(rdx))


@pytest.mark.parametrize("R,L", [(1, 1), (5, 4), (4096, 10), (2 * 3 * 4, 5), (300, 257)])
def test_softmax_vs_oracle(gpu, oracle, R, L):
    rng = np.random.default_rng(R + L)
    x = (rng.standard_normal(R * L) * 4).astype(np.float32)
    dy = rng.standard_normal(R * L).astype(np.float32)
    y, dx = torch.empty(R * L, device="cuda"), torch.empty(R * L, device="cuda")
    ops.softmax_forward(dev(x), y, R, L)
    ry, rdx = np.zeros_like(x), np.zeros_like(x)
    oracle.cnref_softmax_forward(fp(x), fp(ry), R, L)
    ok, msg = close(host(y), ry, 1e-5, 1e-7)
    assert ok, msg
    # backward from the oracle's y: the dot product is summed in the same order
    ops.softmax_backward(dev(ry), dev(dy), dx, R, L)
    oracle.cnref_softmax_backward(fp(ry), fp(dy), fp(rdx), R, L)
    np.testing.assert_array_equal(bits(host(dx)), bits(rdx))
    assert np.allclose(host(y).reshape(L, R).sum(axis=0), 1.0, atol=1e-5)


@pytest.mark.parametrize("from_logits,ls,reduction", [(True, 0.0, "mean"), (True, 0.1, "mean"),
                                                      (False, 0.0, "mean"), (False, 0.2, "sum")])
@pytest.mark.parametrize("B,C", [(7, 3), (4096, 10)])
def test_cce_vs_oracle(gpu, oracle, from_logits, ls, reduction, B, C):
    rng = np.random.default_rng(B * C + int(ls * 10))
    labels = rng.integers(0, C, B)
    T = np.zeros((C, B), np.float32)
    T[labels, np.arange(B)] = 1.0
    t = T.ravel()  # ColMajor [B, C]: column c = class c
    if from_logits:
        p = (rng.standard_normal(B * C) * 2).astype(np.float32)
    else:
        p = rng.dirichlet(np.ones(C), B).astype(np.float32).T.ravel()
    probs, tu = torch.empty(B * C, device="cuda"), torch.empty(B * C, device="cuda")
    loss, g = torch.empty(1, device="cuda"), torch.empty(B * C, device="cuda")
    ops.cce_forward(dev(p), dev(t), probs, tu, loss, B, C, from_logits, ls, reduction)
    red = 0 if reduction == "mean" else 1
    rp, rtu, rg = np.zeros_like(p), np.zeros_like(p), np.zeros_like(p)
    rl = oracle.cnref_cce_forward(fp(p), fp(t), fp(rp), fp(rtu), B, C, int(from_logits), ls, red)
    np.testing.assert_array_equal(bits(host(tu)), bits(rtu))
    ok, msg = close(host(probs), rp, 1e-5, 1e-7)
    assert ok, msg
    assert abs(float(host(loss)[0]) - rl) <= 2e-5 * max(1.0, abs(rl))
    # backward from the oracle's probabilities: elementwise, bit-exact
    ops.cce_backward(dev(rp), dev(rtu), g, B, C, from_logits, reduction)
    oracle.cnref_cce_backward(fp(rp), fp(rtu), fp(rg), B, C, int(from_logits), red)
    np.testing.assert_array_equal(bits(host(g)), bits(rg))


@pytest.mark.parametrize("n", [1, 3, 1000, 1 << 18])
def test_mae_huber_vs_oracle(gpu, oracle, n):
    rng = np.random.default_rng(n + 11)
    p = (rng.standard_normal(n) * 2).astype(np.float32)
    t = (rng.standard_normal(n) * 2).astype(np.float32)
    t[: n // 7] = p[: n // 7]  # exact zeros of the difference
    for reduction, red in (("mean", 0), ("sum", 1)):
        loss, g = torch.empty(1, device="cuda"), torch.empty(n, device="cuda")
        rg = np.zeros(n, np.float32)
        ops.mae_forward(dev(p), dev(t), loss, reduction)
        rl = oracle.cnref_mae_forward(fp(p), fp(t), n, red)
        assert abs(float(host(loss)[0]) - rl) <= 2e-4 * abs(rl) + 1e-7
        ops.mae_backward(dev(p), dev(t), g, reduction)
        oracle.cnref_mae_backward(fp(p), fp(t), fp(rg), n, red)
        np.testing.assert_array_equal(bits(host(g)), bits(rg))
        for delta in (0.5, 1.0, 3.0):
            ops.huber_forward(dev(p), dev(t), loss, delta, reduction)
            rl = oracle.cnref_huber_forward(fp(p), fp(t), n, delta, red)
            assert abs(float(host(loss)[0]) - rl) <= 2e-4 * abs(rl) + 1e-7
            ops.huber_backward(dev(p), dev(t), g, delta, reduction)
            oracle.cnref_huber_backward(fp(p), fp(t), fp(rg), n, delta, red)
            np.testing.assert_array_equal(bits(host(g)), bits(rg))


@pytest.mark.parametrize("kind", ["sgd", "momentum", "adagrad", "rmsprop"])
def test_optimizers_exact(gpu, oracle, kind):
    """Three updates of four tensors (sizes off every block multiple) in one
    launch each, against the oracle's host loops: bit-identical."""
    rng = np.random.default_rng(len(kind))
    sizes = [1, 1000, 2049, 70001]
    lr, hyper, eps = 0.01, (0.9 if kind in ("momentum", "rmsprop") else 0.0), 1e-8
    Ws = [rng.standard_normal(s).astype(np.float32) for s in sizes]
    dW = [dev(w) for w in Ws]
    dS = [torch.zeros(s, device="cuda") for s in sizes] if kind != "sgd" else [None] * len(sizes)
    rS = [np.zeros(s, np.float32) for s in sizes]
    for step in range(3):
        gs = [(rng.standard_normal(s) * (step + 1)).astype(np.float32) for s in sizes]
        ops.optimizer_step_multi(kind, [(w, dev(g), st) for w, g, st in zip(dW, gs, dS)], lr, hyper, eps)
        for w, g, st in zip(Ws, gs, rS):
            if kind == "sgd":
                oracle.cnref_sgd_step(fp(w), fp(g), w.size, lr)
            elif kind == "momentum":
                oracle.cnref_momentum_step(fp(w), fp(g), fp(st), w.size, lr, hyper)
            elif kind == "adagrad":
                oracle.cnref_adagrad_step(fp(w), fp(g), fp(st), w.size, lr, eps)
            else:
                oracle.cnref_rmsprop_step(fp(w), fp(g), fp(st), w.size, lr, hyper, eps)
    for w, rw in zip(dW, Ws):
        np.testing.assert_array_equal(bits(host(w)), bits(rw))
    if kind != "sgd":
        for s, rs in zip(dS, rS):
            np.testing.assert_array_equal(bits(host(s)), bits(rs))


def _dropout_mask_host(n, p, seed, offset):
    """The documented generator: keep entry i when u < 1 - p, u = top 24
    bits of splitmix64(seed + (offset + i) * golden) / 2^24."""
    M = (1 << 64) - 1
    keep = np.float32(1.0) - np.float32(p)
    out = np.zeros(n, np.uint8)
    for i in range(n):
        z = (seed + (offset + i) * 0x9E3779B97F4A7C15) & M
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
        z ^= z >> 31
        u = np.float32(z >> 40) * np.float32(1.0 / 16777216.0)
        out[i] = 1 if u < keep else 0
    return out


@pytest.mark.parametrize("p", [0.0, 0.3, 0.5, 0.9])
def test_dropout(gpu, oracle, p):
    n, seed, offset = 200_000, 1234567, 77
    rng = np.random.default_rng(int(p * 10))
    x, dy = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    y, mask, dx = torch.empty(n, device="cuda"), torch.empty(n, dtype=torch.uint8, device="cuda"), \
        torch.empty(n, device="cuda")
    ops.dropout_forward(dev(x), y, mask, p, seed, offset)
    ops.dropout_backward(dev(dy), mask, dx, p)
    m = host(mask)
    np.testing.assert_array_equal(m[:2000], _dropout_mask_host(2000, p, seed, offset))
    kept = m.mean()
    sd = np.sqrt(p * (1 - p) / n)
    assert abs(kept - (1 - p)) <= 6 * sd + 1e-9, f"kept fraction {kept} for p={p}"
    scale = float(np.float32(1.0) / (np.float32(1.0) - np.float32(p)))
    ry, rdx = np.zeros_like(x), np.zeros_like(x)
    oracle.cnref_dropout_apply(fp(x), fp(m.astype(np.float32)), fp(ry), n, scale)
    oracle.cnref_dropout_apply(fp(dy), fp(m.astype(np.float32)), fp(rdx), n, scale)
    np.testing.assert_array_equal(bits(host(y)), bits(ry))
    np.testing.assert_array_equal(bits(host(dx)), bits(rdx))
    # a different offset gives a different mask; the same (seed, offset) the same
    m2 = torch.empty(n, dtype=torch.uint8, device="cuda")
    ops.dropout_forward(dev(x), y, m2, p, seed, offset)
    np.testing.assert_array_equal(host(m2), m)
    if 0 < p:
        ops.dropout_forward(dev(x), y, m2, p, seed, offset + n)
        assert (host(m2) != m).any()


@pytest.mark.parametrize("N,C,H,W", [(1, 1, 2, 2), (3, 4, 5, 6), (256, 64, 8, 8), (7, 3, 1, 9)])
def test_global_pools_exact(gpu, oracle, N, C, H, W):
    rng = np.random.default_rng(N + C + H + W)
    X = rng.integers(-3, 4, N * C * H * W).astype(np.float32)  # ties: the first max must win
    X += (rng.standard_normal(X.size) * (rng.random(X.size) < 0.3)).astype(np.float32)
    dY = rng.standard_normal(N * C).astype(np.float32)
    Y, dX = torch.empty(N * C, device="cuda"), torch.full((X.size,), 9.0, device="cuda")
    ops.global_avgpool_forward(dev(X), Y, N, C, H, W)
    ops.global_avgpool_backward(dev(dY), dX, N, C, H, W)
    rY, rdX = np.zeros(N * C, np.float32), np.zeros_like(X)
    oracle.cnref_global_avgpool_forward(fp(X), fp(rY), N, C, H, W)
    oracle.cnref_global_avgpool_backward(fp(dY), fp(rdX), N, C, H, W)
    np.testing.assert_array_equal(bits(host(Y)), bits(rY))
    np.testing.assert_array_equal(bits(host(dX)), bits(rdX))
    ah, aw = torch.empty(N * C, dtype=torch.int32, device="cuda"), torch.empty(N * C, dtype=torch.int32,
                                                                              device="cuda")
    dX.fill_(9.0)
    ops.global_maxpool_forward(dev(X), Y, ah, aw, N, C, H, W)
    ops.global_maxpool_backward(dev(dY), ah, aw, dX, N, C, H, W)
    rah, raw = np.zeros(N * C, np.int32), np.zeros(N * C, np.int32)
    oracle.cnref_global_maxpool_forward(fp(X), fp(rY), ip(rah), ip(raw), N, C, H, W)
    oracle.cnref_global_maxpool_backward(fp(dY), ip(rah), ip(raw), fp(rdX), N, C, H, W)
    np.testing.assert_array_equal(bits(host(Y)), bits(rY))
    np.testing.assert_array_equal(host(ah), rah)
    np.testing.assert_array_equal(host(aw), raw)
    np.testing.assert_array_equal(bits(host(dX)), bits(rdX))


@pytest.mark.parametrize("B,S,I,H", [(3, 5, 4, 8), (1, 1, 3, 6), (16, 12, 32, 64), (64, 32, 128, 256)])
def test_rnn_vs_oracle(gpu, oracle, B, S, I, H):
    print(f"[rnn] B={B} S={S} I={I} H={H}", flush=True)
    oracle.cnref_set_threads(16)
    rng = np.random.default_rng(B * S + I + H)
    BS = B * S
    X = rng.standard_normal(BS * I).astype(np.float32)
    Wih = rng.uniform(-np.sqrt(6 / (I + H)), np.sqrt(6 / (I + H)), I * H).astype(np.float32)
    Whh = rng.uniform(-np.sqrt(3 / H), np.sqrt(3 / H), H * H).astype(np.float32)
    b = (rng.standard_normal(H) * 0.1).astype(np.float32)
    dY = (rng.standard_normal(BS * H) * 1e-2).astype(np.float32)
    Y = torch.empty(BS * H, device="cuda")
    ops.rnn_forward(dev(X), dev(Wih), dev(Whh), dev(b), Y, B, S, I, H)
    rY = np.zeros(BS * H, np.float32)
    oracle.cnref_rnn_forward(fp(X), fp(Wih), fp(Whh), fp(b), fp(rY), B, S, I, H)
    ok, msg = close(host(Y), rY, 1e-4, 2e-5)
    assert ok, f"Y: {msg}"
    # backward on the oracle's own forward, so forward rounding does not leak in
    gWih, gWhh, gb, dX = (torch.empty(I * H, device="cuda"), torch.empty(H * H, device="cuda"),
                          torch.empty(H, device="cuda"), torch.empty(BS * I, device="cuda"))
    ops.rnn_backward(dev(X), dev(Wih), dev(Whh), dev(rY), dev(dY), gWih, gWhh, gb, dX, B, S, I, H)
    rgWih, rgWhh, rgb, rdX = (np.zeros(I * H, np.float32), np.zeros(H * H, np.float32),
                              np.zeros(H, np.float32), np.zeros(BS * I, np.float32))
    oracle.cnref_rnn_backward(fp(X), fp(Wih), fp(Whh), fp(rY), fp(dY), fp(rgWih), fp(rgWhh), fp(rgb), fp(rdX),
                              B, S, I, H)
    dTabs = np.full(BS * H, np.abs(dY).mean() * 4, np.float32)
    m_ih = gemm_mag(oracle, 1, 0, I, H, BS, X, BS, dTabs, BS, I)
    m_hh = gemm_mag(oracle, 1, 0, H, H, BS, np.abs(rY), BS, dTabs, BS, H)
    m_b = gemm_mag(oracle, 1, 0, 1, H, BS, np.ones(BS, np.float32), BS, dTabs, BS, 1)
    m_dx = gemm_mag(oracle, 0, 1, BS, I, H, dTabs, BS, Wih, I, BS)
    for got, want, mag, name in [(host(gWih), rgWih, m_ih, "grad_W_ih"), (host(gWhh), rgWhh, m_hh, "grad_W_hh"),
                                 (host(gb), rgb, m_b, "grad_b"), (host(dX), rdX, m_dx, "dX")]:
        ok, msg = close_mag(got, want, mag, 1e-4, 1e-5)
        assert ok, f"{name}: {msg}"
