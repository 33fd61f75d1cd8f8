"""Layers::Residual on the GPU (A23): the reference's residual benchmark
network (benchmarks/residual_benckmark.cpp:104-152) built by the C++
session from Linear + Residual + ReLU + SoftmaxCrossEntropy + Adam, against
the oracle composition (oracle/resnet.py, whose Residual restatement is
pinned by tests/test_oracle_residual.py) on identical inputs and weights.

Both shortcut kinds run: identity (every block W -> W) and a projection (the
last block maps W -> last_width != W, so Residual builds its bias-free
"ResProj" Linear, residual.cpp:31-36).

Bars: one step -- loss rel 1e-4; every gradient elementwise within
1e-5 + 1e-4 max(|ref|, |X|^T|dA|/sqrt(B)), the per-element magnitude of
each weight-gradient contraction (its bias analogue for biases); updated
weights within the same bound except where the gradient itself is within
tolerance of 0 (Adam's step 1 is -lr sign(g)).  Twenty steps -- the loss
within rel 1e-3 at every step and each parameter within rel 1e-3 in norm
(or 2x the oracle's own drift across four other valid evaluation orders).
"""
import os

import numpy as np
import pytest

from cppnet_amd import trainer
from oracle.resnet import OracleResNet
from oracle_lib import close, close_mag, gemm_mag

pytestmark = pytest.mark.gpu

CASES = {"identity": dict(last_width=0), "projection": dict(last_width=96)}


@pytest.fixture(scope="module")
def oracle_mt(oracle):
    oracle.cnref_set_threads(min(16, os.cpu_count() or 1))
    return oracle


def _cfg(kind, batch=128):
    return trainer.ResNetConfig(f"resnet {kind}", 24, 160, 3, 5, batch, **CASES[kind])


def _mags(oracle, ref, cfg):
    """|X|^T |dA| / sqrt(B) per weight-gradient element, |1|^T|dA|/sqrt(B) per bias."""
    B = cfg.batch
    mags = [None] * len(ref.params)
    for k, (x, dA, I, O) in ref.trace.items():
        mags[k] = gemm_mag(oracle, 1, 0, I, O, B, x, B, dA, B, I)
        if k + 1 < len(mags) and ref.params[k + 1].size == O and ref.shapes[k + 1] == (O,):
            mags[k + 1] = gemm_mag(oracle, 1, 0, 1, O, B, np.ones(B, np.float32), B, dA, B, 1)
    assert all(m is not None for m in mags)
    return mags


@pytest.mark.parametrize("kind", sorted(CASES))
def test_resnet_one_step(gpu, oracle_mt, kind):
    cfg = _cfg(kind)
    print(f"[residual] {cfg.name}: one step", flush=True)
    params, X, Y = trainer.synthetic_resnet(cfg, np.random.default_rng(31))
    sess = trainer.Session(cfg)
    assert sess.num_params() == len(params)
    sess.set_params(params)
    sess.set_batch(X, Y)
    ref = OracleResNet(cfg, oracle_mt)
    ref.set_params(params)
    loss_gpu = sess.forward_backward()
    g_gpu = sess.get_grads()
    sess.update()
    loss_ref = ref.step(X, Y)
    ok, msg = close([loss_gpu], [loss_ref], 1e-4, 1e-5)
    assert ok, f"loss: {msg}"
    mags = _mags(oracle_mt, ref, cfg)
    for k, (a, b, m) in enumerate(zip(g_gpu, ref.last_grads, mags)):
        ok, msg = close_mag(a, b, m, 1e-4, 1e-5)
        assert ok, f"grad of param {k} {ref.shapes[k]}: {msg}"
    for k, (a, b, g, m) in enumerate(zip(sess.get_params(), ref.get_params(), ref.last_grads, mags)):
        err = np.abs(a.astype(np.float64) - b)
        bad = err > 1e-5 + 1e-4 * np.abs(b)
        ill = np.abs(g) <= 1e-5 + 1e-4 * np.maximum(np.abs(g), m)
        assert not (bad & ~ill).any(), f"param {k}: updated weights differ where |g| is well conditioned"
    sess.close()


def _rel(a, b):
    return float(np.linalg.norm(a.astype(np.float64) - b) / max(np.linalg.norm(b), 1e-30))


# (double accumulation, fp32 sum order) of the oracle's alternative
# evaluation orders: double accumulation rounded once per element, fp32 in
# descending order, fp32 in 32-wide chunks, fp32 in 8 strided partials
ORDERS = [(1, 0), (0, 1), (0, 2), (0, 3)]


def _oracle_run(cfg, oracle, seed, steps, double, order):
    rng = np.random.default_rng(seed)
    params, _, _ = trainer.synthetic_resnet(cfg, rng)
    ref = OracleResNet(cfg, oracle)
    ref.set_params(params)
    oracle.cnref_set_accumulate_double(double)
    oracle.cnref_set_sum_order(order)
    try:
        losses = [ref.step(*trainer.synthetic_resnet(cfg, rng)[1:]) for _ in range(steps)]
    finally:
        oracle.cnref_set_accumulate_double(0)
        oracle.cnref_set_sum_order(0)
    return ref.get_params(), np.array(losses)


@pytest.mark.parametrize("kind", sorted(CASES))
def test_resnet_multi_step(gpu, oracle_mt, kind):
    """The drift of a parameter is the largest distance from the fp32 oracle
    of the oracle's own runs under the four other evaluation orders.  The
    identity network is rounding-sensitive: a bias-gradient sum that nearly
    cancels is turned into a +-lr Adam step by its sign (adam.cpp:98-133),
    so the fp32 orders alone part by ~1e-3 (descending) to ~3e-3 (chunked)
    on the first two biases after 20 steps, while double accumulation moves
    them by only ~6e-6; every order is a valid fp32 evaluation, so the bar
    is max(1e-3, 2 x that drift)."""
    cfg = _cfg(kind, batch=64)
    steps, seed = 20, 32
    print(f"[residual] {cfg.name}: {steps} steps", flush=True)
    rng = np.random.default_rng(seed)
    params, _, _ = trainer.synthetic_resnet(cfg, rng)
    sess = trainer.Session(cfg)
    sess.set_params(params)
    ref = OracleResNet(cfg, oracle_mt)
    ref.set_params(params)
    for step in range(steps):
        _, X, Y = trainer.synthetic_resnet(cfg, rng)
        sess.set_batch(X, Y)
        lg, lr_ = sess.step(), ref.step(X, Y)
        assert abs(lg - lr_) <= 1e-3 * abs(lr_) + 1e-6, f"step {step}: loss {lg} vs {lr_}"
    want = ref.get_params()
    runs = [_oracle_run(cfg, oracle_mt, seed, steps, d, o)[0] for d, o in ORDERS]
    for k, (a, b) in enumerate(zip(sess.get_params(), want)):
        rel = _rel(a, b)
        drift = max(_rel(r[k], b) for r in runs)
        print(f"[residual] {kind} param {k}: rel {rel:.3g} drift {drift:.3g}")
        assert rel <= max(1e-3, 2.0 * drift), f"param {k}: relative norm error {rel:.3g} (drift {drift:.3g})"
    sess.close()


def test_resnet_grads_accumulate_until_zero_grad(gpu):
    """Linear grads inside the Residual accumulate across backward calls and are
    cleared by zero_grad (linear.cpp:346-352, residual.cpp:143-156): two
    forward_backward calls without an update -> each call zero_grads first,
    so the grads equal one call's."""
    cfg = _cfg("projection", batch=16)
    params, X, Y = trainer.synthetic_resnet(cfg, np.random.default_rng(33))
    sess = trainer.Session(cfg)
    sess.set_params(params)
    sess.set_batch(X, Y)
    sess.forward_backward()
    g1 = sess.get_grads()
    sess.forward_backward()
    g2 = sess.get_grads()
    assert all(np.array_equal(a, b) for a, b in zip(g1, g2))
    sess.close()
