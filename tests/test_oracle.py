"""Pins the CPU oracle (CPU only, no GPU).

Each oracle function is checked against (1) the known answers of the
reference's own tests (tests/golden/known_answers.json), and (2) what the
mathematics fixes independently of the oracle's code: float64 torch autograd
on logical (row-major) tensors for gradients, closed forms for Adam, and
float64 brute force for the GEMM in every transpose combination.  A swapped
operand, a dropped term or a ColMajor/RowMajor index slip fails (2) even when
it survives (1).
"""
import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle_lib import close, colmajor, fp, from_colmajor

GOLD = json.loads((Path(__file__).parent / "golden" / "known_answers.json").read_text())["cases"]


@pytest.fixture(params=[0, 1], ids=["eigen", "cpu_loops"])
def linear_mode(oracle, request):
    """The oracle's Linear as the cpu-eigen contraction (default) or as the
    reference's "cpu" device loops (cnref_set_cpu_loops, used for timing the
    reference's "cpu" leg): both are held to the same checks."""
    oracle.cnref_set_cpu_loops(request.param)
    yield request.param
    oracle.cnref_set_cpu_loops(0)


def _cases(op):
    return [c for c in GOLD if c["op"] == op]


def _shape(rows):
    a = np.asarray(rows)
    return a.shape if a.ndim == 2 else (1, a.shape[0])


# ---------------------------------------------------------------- known answers
@pytest.mark.parametrize("case", _cases("linear_forward"), ids=lambda c: c["source"])
def test_known_linear_forward(oracle, case, linear_mode):
    B, I = _shape(case["X"])
    O = np.asarray(case["W"]).shape[1]
    X, W = colmajor(case["X"]), colmajor(case["W"])
    b = None if case["b"] is None else np.asarray(case["b"], np.float32)
    Y = np.zeros(B * O, np.float32)
    oracle.cnref_linear_forward(fp(X), fp(W), fp(b), fp(Y), B, I, O)
    np.testing.assert_allclose(from_colmajor(Y, B, O), case["expected"], atol=case["tol"])


def test_known_relu_backward(oracle):
    (case,) = _cases("relu_backward")
    R, Cc = _shape(case["X"])
    x, dy = colmajor(case["X"]), colmajor(case["dY"])
    y, dx = np.zeros_like(x), np.zeros_like(x)
    oracle.cnref_relu_forward(fp(x), fp(y), x.size)
    oracle.cnref_relu_backward(fp(y), fp(dy), fp(dx), x.size)
    got = from_colmajor(dx, R, Cc)
    xl = np.asarray(case["X"])
    assert np.all(got[xl > 0] > 0) and np.all(np.abs(got[xl <= 0]) <= case["tol"])
    np.testing.assert_array_equal(got, case["exact"])


@pytest.mark.parametrize("case", _cases("sigmoid_forward"), ids=lambda c: c["source"])
def test_known_sigmoid_forward(oracle, case):
    x = colmajor(case["X"])
    y = np.zeros_like(x)
    oracle.cnref_sigmoid_forward(fp(x), fp(y), x.size)
    R, Cc = _shape(case["X"])
    np.testing.assert_allclose(from_colmajor(y, R, Cc), case["expected"], atol=case["tol"])


def test_known_sigmoid_backward(oracle):
    (case,) = _cases("sigmoid_backward")
    x, dy = colmajor(case["X"]), colmajor(case["dY"])
    y, dx = np.zeros_like(x), np.zeros_like(x)
    oracle.cnref_sigmoid_forward(fp(x), fp(y), x.size)
    oracle.cnref_sigmoid_backward(fp(y), fp(dy), fp(dx), x.size)
    R, Cc = _shape(case["X"])
    np.testing.assert_allclose(from_colmajor(dx, R, Cc), case["expected"], atol=case["tol"])


@pytest.mark.parametrize("case", _cases("bce_forward"), ids=lambda c: c["source"])
def test_known_bce_forward(oracle, case):
    p, t = colmajor(case["P"]), colmajor(case["T"])
    loss = oracle.cnref_bce_forward(fp(p), fp(t), p.size, 0)
    if "expected" in case:
        assert abs(loss - case["expected"]) <= case["tol"]
    if "exact" in case:
        assert abs(loss - case["exact"]) <= case["tol"] + 1e-6 * abs(case["exact"])


def test_known_bce_backward(oracle):
    (case,) = _cases("bce_backward")
    p, t = colmajor(case["P"]), colmajor(case["T"])
    g = np.zeros_like(p)
    oracle.cnref_bce_backward(fp(p), fp(t), fp(g), p.size, 0)
    assert g[0] < 0
    np.testing.assert_allclose(g, np.ravel(case["exact"]), atol=case["tol"])


@pytest.mark.parametrize("case", _cases("mse_forward"), ids=lambda c: c["source"])
def test_known_mse_forward(oracle, case):
    p, t = colmajor(case["P"]), colmajor(case["T"])
    assert abs(oracle.cnref_mse_forward(fp(p), fp(t), p.size, 0) - case["expected"]) <= case["tol"]


def test_known_mse_backward(oracle):
    (case,) = _cases("mse_backward")
    p, t = colmajor(case["P"]), colmajor(case["T"])
    g = np.zeros_like(p)
    oracle.cnref_mse_backward(fp(p), fp(t), fp(g), p.size, 0)
    assert np.all(g > 0)
    np.testing.assert_allclose(g, np.ravel(case["exact"]), atol=case["tol"])


@pytest.mark.parametrize("case", _cases("softmax_ce_forward"), ids=lambda c: c["source"])
def test_known_softmax_ce_forward(oracle, case):
    B, Cc = _shape(case["Z"])
    z, t = colmajor(case["Z"]), colmajor(case["T"])
    sm = np.zeros_like(z)
    loss = oracle.cnref_softmax_ce_forward(fp(z), fp(t), fp(sm), B, Cc, 0)
    assert abs(loss - case["exact"]) <= case["tol"] * max(1.0, abs(case["exact"]))
    assert eval(case["check"], {"loss": loss})


def test_known_softmax_ce_backward(oracle):
    (case,) = _cases("softmax_ce_backward")
    B, Cc = _shape(case["Z"])
    z, t = colmajor(case["Z"]), colmajor(case["T"])
    sm, g = np.zeros_like(z), np.zeros_like(z)
    oracle.cnref_softmax_ce_forward(fp(z), fp(t), fp(sm), B, Cc, 0)
    oracle.cnref_softmax_ce_backward(fp(sm), fp(t), fp(g), B, Cc, 0)
    got = from_colmajor(g, B, Cc)
    np.testing.assert_allclose(got, case["expected"], atol=case["tol"])
    np.testing.assert_allclose(got, case["exact"], atol=1e-6)


def test_known_adam_first_step(oracle):
    (case,) = _cases("adam_first_step")
    W = np.asarray(case["W"], np.float32)
    g = np.asarray(case["G"], np.float32)
    m, v = np.zeros_like(W), np.zeros_like(W)
    bc1 = oracle.cnref_bias_correction(case["beta1"], 1)
    bc2 = oracle.cnref_bias_correction(case["beta2"], 1)
    oracle.cnref_adam_step(fp(W), fp(g), fp(m), fp(v), W.size, case["lr"], case["beta1"],
                           case["beta2"], case["eps"], bc1, bc2)
    np.testing.assert_allclose(W, case["exact"], atol=case["tol"])


# ---------------------------------------------------------------- GEMM brute force
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (5, 7, 3), (33, 17, 65), (8, 1, 40), (3, 4, 0)])
def test_gemm_brute_force(oracle, ta, tb, M, N, K):
    rng = np.random.default_rng(M * 1000 + N * 10 + K + 7 * ta + 3 * tb)
    Al = rng.standard_normal((M, K)).astype(np.float32)  # logical op(A)
    Bl = rng.standard_normal((K, N)).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    lda = (K if ta else M) + 2
    ldb = (N if tb else K) + 1
    ldc = M + 3
    # store op(A) so that op(A)(m,k) is read as specified in cnref.h
    A = np.zeros(lda * (M if ta else K) + 1, np.float32)
    for m in range(M):
        for k in range(K):
            A[(k + lda * m) if ta else (m + lda * k)] = Al[m, k]
    B = np.zeros(ldb * (K if tb else N) + 1, np.float32)
    for k in range(K):
        for n in range(N):
            B[(n + ldb * k) if tb else (k + ldb * n)] = Bl[k, n]
    C = np.zeros(ldc * N, np.float32)
    for m in range(M):
        for n in range(N):
            C[m + ldc * n] = C0[m, n]
    alpha, beta = 0.75, -0.5
    oracle.cnref_gemm_f32(ta, tb, M, N, K, alpha, fp(A), lda, fp(B), ldb, beta, fp(C), ldc,
                          fp(bias), 1)
    want = np.maximum(alpha * (Al.astype(np.float64) @ Bl) + beta * C0 + bias, 0.0)
    got = np.array([[C[m + ldc * n] for n in range(N)] for m in range(M)])
    ok, msg = close(got, want, rtol=1e-5, atol=1e-5)
    assert ok, msg


# ---------------------------------------------------------------- float64 autograd
def _t64(a):
    return torch.tensor(np.asarray(a, np.float64), requires_grad=True)


@pytest.mark.parametrize("B,I,O", [(4, 3, 5), (64, 30, 17), (7, 1, 1)])
def test_linear_backward_vs_autograd(oracle, B, I, O, linear_mode):
    rng = np.random.default_rng(B + I + O)
    Xl = rng.standard_normal((B, I)).astype(np.float32)
    Wl = rng.standard_normal((I, O)).astype(np.float32)
    bl = rng.standard_normal(O).astype(np.float32)
    dYl = rng.standard_normal((B, O)).astype(np.float32)
    gW0 = rng.standard_normal((I, O)).astype(np.float32)  # pre-existing grads: accumulated into
    gb0 = rng.standard_normal(O).astype(np.float32)

    X, W, dY = colmajor(Xl), colmajor(Wl), colmajor(dYl)
    Y = np.zeros(B * O, np.float32)
    oracle.cnref_linear_forward(fp(X), fp(W), fp(bl), fp(Y), B, I, O)
    gW, gb, dX = colmajor(gW0), gb0.copy(), np.zeros(B * I, np.float32)
    oracle.cnref_linear_backward(fp(X), fp(W), fp(dY), fp(gW), fp(gb), fp(dX), B, I, O, 1, 1)

    xt, wt, bt = _t64(Xl), _t64(Wl), _t64(bl)
    yt = xt @ wt + bt
    yt.backward(torch.tensor(dYl, dtype=torch.float64))
    for got, want, name in [(from_colmajor(Y, B, O), yt.detach().numpy(), "Y"),
                            (from_colmajor(gW, I, O), gW0 + wt.grad.numpy(), "gW"),
                            (gb, gb0 + bt.grad.numpy(), "gb"),
                            (from_colmajor(dX, B, I), xt.grad.numpy(), "dX")]:
        ok, msg = close(got, want, rtol=1e-5, atol=1e-5)
        assert ok, f"{name}: {msg}"


def test_linear_not_trainable_skips_param_grads(oracle, linear_mode):
    B, I, O = 3, 2, 4
    X = np.ones(B * I, np.float32)
    W = np.ones(I * O, np.float32)
    dY = np.ones(B * O, np.float32)
    gW = np.full(I * O, 7.0, np.float32)
    gb = np.full(O, 7.0, np.float32)
    dX = np.zeros(B * I, np.float32)
    oracle.cnref_linear_backward(fp(X), fp(W), fp(dY), fp(gW), fp(gb), fp(dX), B, I, O, 0, 1)
    assert np.all(gW == 7.0) and np.all(gb == 7.0)
    assert np.all(dX == O)  # dX is computed even when frozen (linear.cpp:357)


def test_mlp_step_cpu_loops_matches_eigen(oracle):
    """A whole MLP train step (forward, softmax-CE, backward, Adam) with the
    Linear layers as the "cpu" device loops agrees with the cpu-eigen step to
    fp32 rounding: the loops change only the order of the fp32 sums."""
    from cppnet_amd import trainer
    from oracle.mlp import OracleMLP
    cfg = trainer.MLPConfig("MLP 33-70-48-10 softmax-CE", [33, 70, 48, 10], "relu", "none", "softmax_ce", 96)
    params, X, Y = trainer.synthetic_mlp(cfg, np.random.default_rng(4))
    runs = []
    for loops in (0, 1):
        oracle.cnref_set_cpu_loops(loops)
        try:
            ref = OracleMLP(cfg, oracle)
            ref.set_params(params)
            losses = [ref.step(X, Y) for _ in range(2)]
            runs.append((losses, ref.get_params()))
        finally:
            oracle.cnref_set_cpu_loops(0)
    (l0, p0), (l1, p1) = runs
    assert np.allclose(l0, l1, rtol=1e-5, atol=0), (l0, l1)
    for k, (a, b) in enumerate(zip(p0, p1)):
        ok, msg = close(b, a, rtol=1e-4, atol=1e-6)
        assert ok, f"parameter {k}: {msg}"


@pytest.mark.parametrize("name", ["relu", "sigmoid", "tanh"])
def test_activation_grads_vs_autograd(oracle, name):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(257) * 3).astype(np.float32)
    x[:3] = [0.0, 600.0, -600.0]  # relu kink (gated), sigmoid clamp
    dy = rng.standard_normal(257).astype(np.float32)
    y, dx = np.zeros_like(x), np.zeros_like(x)
    getattr(oracle, f"cnref_{name}_forward")(fp(x), fp(y), x.size)
    getattr(oracle, f"cnref_{name}_backward")(fp(y), fp(dy), fp(dx), x.size)
    xt = _t64(x)
    if name == "sigmoid":
        yt = torch.sigmoid(torch.clamp(xt, -500, 500))
    else:
        yt = getattr(torch, name)(xt)
    yt.backward(torch.tensor(dy, dtype=torch.float64))
    want_dx = xt.grad.numpy().copy()
    if name == "sigmoid":
        # the reference differentiates through s(1-s) of the (clamped) output,
        # not through the clamp: s(1-s) is nonzero beyond +-500 only as 0.
        s = yt.detach().numpy()
        want_dx = dy * s * (1 - s)
    ok, msg = close(y, yt.detach().numpy(), rtol=2e-6, atol=1e-7)
    assert ok, msg
    ok, msg = close(dx, want_dx, rtol=1e-5, atol=1e-6)
    assert ok, msg


def test_bce_vs_autograd(oracle):
    rng = np.random.default_rng(5)
    p = rng.uniform(0.02, 0.98, 300).astype(np.float32)
    p[:2] = [0.0, 1.0]  # clipped to [1e-7, 1-1e-7]
    t = (rng.uniform(size=300) < 0.5).astype(np.float32)
    g = np.zeros_like(p)
    loss = oracle.cnref_bce_forward(fp(p), fp(t), p.size, 0)
    oracle.cnref_bce_backward(fp(p), fp(t), fp(g), p.size, 0)
    pc = np.clip(p.astype(np.float64), 1e-7, 1 - 1e-7)
    pt = torch.tensor(pc, requires_grad=True)
    lt = torch.nn.functional.binary_cross_entropy(pt, torch.tensor(t, dtype=torch.float64))
    lt.backward()
    assert abs(loss - lt.item()) <= 1e-5 * abs(lt.item())
    ok, msg = close(g, pt.grad.numpy(), rtol=1e-5, atol=1e-9)
    assert ok, msg
    # sum reduction: n times the mean's gradient
    oracle.cnref_bce_backward(fp(p), fp(t), fp(g), p.size, 1)
    ok, msg = close(g, pt.grad.numpy() * p.size, rtol=1e-5, atol=1e-7)
    assert ok, msg


def test_mse_vs_autograd(oracle):
    rng = np.random.default_rng(6)
    p = rng.standard_normal(128).astype(np.float32)
    t = rng.standard_normal(128).astype(np.float32)
    g = np.zeros_like(p)
    loss = oracle.cnref_mse_forward(fp(p), fp(t), p.size, 0)
    oracle.cnref_mse_backward(fp(p), fp(t), fp(g), p.size, 0)
    pt = torch.tensor(p.astype(np.float64), requires_grad=True)
    lt = torch.nn.functional.mse_loss(pt, torch.tensor(t, dtype=torch.float64))
    lt.backward()
    assert abs(loss - lt.item()) <= 1e-5 * lt.item()
    ok, msg = close(g, pt.grad.numpy(), rtol=1e-5, atol=1e-9)
    assert ok, msg


@pytest.mark.parametrize("B,Cc", [(1, 3), (37, 10), (64, 4)])
def test_softmax_ce_vs_autograd(oracle, B, Cc):
    rng = np.random.default_rng(B * Cc)
    zl = (rng.standard_normal((B, Cc)) * 4).astype(np.float32)
    labels = rng.integers(0, Cc, B)
    tl = np.eye(Cc, dtype=np.float32)[labels]
    z, t = colmajor(zl), colmajor(tl)
    sm, g = np.zeros_like(z), np.zeros_like(z)
    loss = oracle.cnref_softmax_ce_forward(fp(z), fp(t), fp(sm), B, Cc, 0)
    oracle.cnref_softmax_ce_backward(fp(sm), fp(t), fp(g), B, Cc, 0)
    zt = torch.tensor(zl.astype(np.float64), requires_grad=True)
    lt = torch.nn.functional.cross_entropy(zt, torch.tensor(labels))
    lt.backward()
    assert abs(loss - lt.item()) <= 1e-5 * max(1.0, lt.item())
    ok, msg = close(from_colmajor(sm, B, Cc), torch.softmax(zt, 1).detach().numpy(), 1e-5, 1e-7)
    assert ok, msg
    ok, msg = close(from_colmajor(g, B, Cc), zt.grad.numpy(), rtol=1e-5, atol=1e-8)
    assert ok, msg


def test_adam_two_steps_vs_float64(oracle):
    rng = np.random.default_rng(9)
    n = 1000
    W = rng.standard_normal(n).astype(np.float32)
    m, v = np.zeros(n, np.float32), np.zeros(n, np.float32)
    Wd, md, vd = W.astype(np.float64), np.zeros(n), np.zeros(n)
    lr, b1, b2, eps = 1e-3, 0.9, 0.999, 1e-8
    for t in (1, 2, 3):
        g = rng.standard_normal(n).astype(np.float32)
        bc1 = oracle.cnref_bias_correction(b1, t)
        bc2 = oracle.cnref_bias_correction(b2, t)
        assert abs(bc1 - (1 - 0.9 ** t)) < 1e-6 and abs(bc2 - (1 - 0.999 ** t)) < 1e-6
        oracle.cnref_adam_step(fp(W), fp(g), fp(m), fp(v), n, lr, b1, b2, eps, bc1, bc2)
        md = b1 * md + (1 - b1) * g
        vd = b2 * vd + (1 - b2) * g.astype(np.float64) ** 2
        Wd = Wd - lr * (md / (1 - b1 ** t)) / (np.sqrt(vd / (1 - b2 ** t)) + eps)
    ok, msg = close(W, Wd, rtol=1e-6, atol=1e-6)
    assert ok, msg


def test_column_sum(oracle):
    rng = np.random.default_rng(1)
    a = rng.standard_normal((50, 7)).astype(np.float32)
    out = np.ones(7, np.float32)
    oracle.cnref_column_sum(fp(colmajor(a)), fp(out), 50, 7, 1)
    np.testing.assert_allclose(out, 1 + a.sum(0, dtype=np.float64), rtol=1e-5, atol=1e-5)
