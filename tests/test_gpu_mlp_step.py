"""The fused two-launch train step of config 1's model (cnhip_mlp2_bce_adam_step:
Linear -> ReLU -> Linear(., 1) -> Sigmoid, BCE, Adam) against the oracle.

cnt_step takes the fused path for this model.  Step 1 is checked against
the oracle's step 1 from the same weights; step 2 re-anchored: the oracle
loaded with the session's parameters and Adam state (m, v, t) after step 1
runs step 2 on the same batch.  The GPU's loss, gradients and updated
parameters are held to the one-step bars of tests/test_gpu_model.py
(contractions magnitude-aware, the ReLU-mask allowance, Adam's
sign-sensitive updates where the gradient lies within its bar of 0).  The
per-block sums over the batch are an evaluation order of their own, so the
bars, not bit-equality, are the check."""
import ctypes as C
import os

import numpy as np
import pytest

from cppnet_amd import _capi, trainer
from model_bars import _grad_mags, _mask_allowance
from oracle.mlp import OracleMLP
from oracle_lib import close, close_mag

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def oracle_mt(oracle):
    oracle.cnref_set_threads(min(16, os.cpu_count() or 1))
    return oracle


def _kernels_run(fn):
    lib = _capi.load()
    _capi.check(lib.cnhip_hbm_timing_enable(1))
    try:
        fn()
        return {r["kernel"] for r in _capi.hbm_timing_rows()}
    finally:
        _capi.check(lib.cnhip_hbm_timing_enable(0))


def _check_step(sess, ref, cfg, oracle, p0, X, Y, t_before):
    """One fused session step against one oracle step from the same state."""
    loss_box = []
    ran = _kernels_run(lambda: loss_box.append(sess.step()))
    assert {"mlp2_bce_part_kernel", "mlp2_bce_adam_kernel"} <= ran, f"fused step not taken: {sorted(ran)}"
    loss_gpu, loss_ref = loss_box[0], ref.step(X, Y)
    ok, msg = close([loss_gpu], [loss_ref], 1e-4, 1e-5)
    assert ok, f"loss: {msg}"
    mags = _grad_mags(oracle, ref, cfg)
    allow = _mask_allowance(oracle, ref, cfg, p0)
    for k, (a, b, mag, al) in enumerate(zip(sess.get_grads(), ref.last_grads, mags, allow)):
        ok, msg = close_mag(a, b, mag, 1e-4, 1e-5)
        if not ok:
            err = np.abs(a.astype(np.float64) - b)
            bad = err > 1e-5 + 1e-4 * np.maximum(np.abs(b), mag) + al
            assert not bad.any(), f"grad of param {k}: {int(bad.sum())} outside tolerance + mask allowance ({msg})"
    for k, (a, b, g, mag, al) in enumerate(zip(sess.get_params(), ref.get_params(), ref.last_grads, mags, allow)):
        err = np.abs(a.astype(np.float64) - b)
        bad = err > 1e-5 + 1e-4 * np.abs(b)
        unexplained = bad & (np.abs(g) > 1e-5 + 1e-4 * np.maximum(np.abs(g), mag) + al)
        assert not unexplained.any(), f"param {k}: {int(unexplained.sum())} weights differ where |g| is well conditioned"
    m2, t2 = sess.get_opt_state(0)
    assert t2 == [x + 1 for x in t_before], f"Adam step counts {t2} after {t_before}"
    for k, (a, b) in enumerate(zip(m2, ref.opt.m)):
        g_tol = 1e-5 + 1e-4 * np.maximum(np.abs(ref.last_grads[k]), mags[k]) + allow[k]
        assert (np.abs(a.astype(np.float64) - b) <= (1.0 - cfg.beta1) * g_tol + 1e-6 * np.abs(b) + 1e-12).all(), \
            f"Adam m of param {k}"


def _two_fused_steps(cfg, oracle, params, X1, Y1, X2, Y2):
    """Step 1 against the oracle from the same weights, then step 2 against
    the oracle re-anchored at the session's parameters and Adam state."""
    sess = trainer.Session(cfg)
    try:
        sess.set_params(params)
        ref = OracleMLP(cfg, oracle)
        ref.set_params(params)
        sess.set_batch(X1, Y1)
        _check_step(sess, ref, cfg, oracle, params, X1, Y1, [0, 0, 0, 0])
        p1 = sess.get_params()
        m, t = sess.get_opt_state(0)
        v, _ = sess.get_opt_state(1)
        ref = OracleMLP(cfg, oracle)
        ref.set_params(p1)
        for dst, src in zip(ref.opt.m + ref.opt.v, list(m) + list(v)):
            np.copyto(dst, src)
        ref.opt.t = list(t)
        sess.set_batch(X2, Y2)
        _check_step(sess, ref, cfg, oracle, p1, X2, Y2, t)
    finally:
        sess.close()


@pytest.mark.parametrize("batch", [None, 64])
def test_fused_mlp_step_vs_oracle(gpu, oracle_mt, batch):
    cfg = trainer.mlp_config(1, batch)
    print(f"[mlp-step] config 1 batch {cfg.batch}: two fused steps", flush=True)
    rng = np.random.default_rng(31)
    params, X1, Y1 = trainer.synthetic_mlp(cfg, rng)
    _, X2, Y2 = trainer.synthetic_mlp(cfg, rng)
    _two_fused_steps(cfg, oracle_mt, params, X1, Y1, X2, Y2)


# layer sizes that are not multiples of 4 (the kernel's zero padding of rows
# and columns), the largest sizes, one input, and batches of 1, 3 and 5 blocks
@pytest.mark.parametrize("I,H,B", [(7, 50, 48), (64, 64, 32), (1, 3, 16), (33, 17, 80)])
def test_fused_mlp_step_odd_sizes(gpu, oracle_mt, I, H, B):
    cfg = trainer.MLPConfig(f"MLP {I}-{H}-1 sigmoid BCE", [I, H, 1], "relu", "sigmoid", "bce", B)
    print(f"[mlp-step] {I}-{H}-1 batch {B}: two fused steps", flush=True)
    rng = np.random.default_rng(1000 * I + H)
    params, X1, Y1 = trainer.synthetic_mlp(cfg, rng)
    # biases away from 0 from the first step on
    params[1] = (0.1 * rng.standard_normal(H)).astype(np.float32)
    params[3] = (0.1 * rng.standard_normal(1)).astype(np.float32)
    _, X2, Y2 = trainer.synthetic_mlp(cfg, rng)
    _two_fused_steps(cfg, oracle_mt, params, X1, Y1, X2, Y2)


# models the fused step does not take: a layer wider than 64, or a batch that
# is not a multiple of 16, run layer by layer
@pytest.mark.parametrize("I,H,B", [(30, 65, 64), (65, 8, 64), (30, 64, 40)])
def test_unfused_shapes_run_layer_by_layer(gpu, I, H, B):
    cfg = trainer.MLPConfig(f"MLP {I}-{H}-1 sigmoid BCE", [I, H, 1], "relu", "sigmoid", "bce", B)
    params, X, Y = trainer.synthetic_mlp(cfg, np.random.default_rng(9))
    sess = trainer.Session(cfg)
    try:
        sess.set_params(params)
        sess.set_batch(X, Y)
        box = []
        ran = _kernels_run(lambda: box.append(sess.step()))
        assert "mlp2_bce_part_kernel" not in ran and "mlp2_bce_adam_kernel" not in ran, sorted(ran)
        assert np.isfinite(box[0])
    finally:
        sess.close()


def test_capture_after_fused_steps(gpu):
    """A capture after fused steps runs one layer-by-layer forward + backward
    to size its buffers, then replays the layer-by-layer step: the run stays
    within rounding of a session that never fused."""
    cfg = trainer.mlp_config(1, 64)
    rng = np.random.default_rng(5)
    params, X, Y = trainer.synthetic_mlp(cfg, rng)
    a, b = trainer.Session(cfg), trainer.Session(cfg)
    b.set_fused_step(False)
    for s in (a, b):
        s.set_params(params)
        s.set_batch(X, Y)
        s.step()
        s.step()
    a.capture()
    assert a.has_graph
    for _ in range(3):
        la, lb = a.step(), b.step()
        assert a.has_graph
        assert abs(la - lb) <= 1e-4 * abs(lb) + 1e-6, f"loss {la} (replayed) vs {lb}"
    for k, (pa, pb) in enumerate(zip(a.get_params(), b.get_params())):
        assert np.abs(pa - pb).max() <= 1e-4 * np.abs(pb).max() + 1e-5, f"parameter {k}"
    a.close()
    b.close()


def test_fused_mlp_step_refuses_bad_shapes(gpu):
    lib = _capi.load()
    import torch
    f = lambda n: torch.zeros(n, device="cuda")
    X, Y, W1, b1, W2, b2 = f(48 * 30), f(48), f(30 * 64), f(64), f(64), f(1)
    g = [f(30 * 64), f(64), f(64), f(1)]
    mv = [f(30 * 64), f(64), f(64), f(1)]
    P = (C.c_void_p * 4)(*[t.data_ptr() for t in mv])
    bc = (C.c_float * 4)(0.1, 0.1, 0.1, 0.1)
    loss = f(1)

    def call(B, I, H):
        return lib.cnhip_mlp2_bce_adam_step(X.data_ptr(), Y.data_ptr(), B, I, H, W1.data_ptr(), b1.data_ptr(),
                                            W2.data_ptr(), b2.data_ptr(), *[t.data_ptr() for t in g], P, P, bc, bc,
                                            1e-3, 0.9, 0.999, 1e-8, 0, 0, loss.data_ptr(), None)
    err = lambda: lib.cnhip_last_error().decode()
    assert call(40, 30, 64) != 0 and "multiple of 16" in err()
    assert call(48, 65, 64) != 0 and "layer sizes" in err()
    assert call(48, 30, 64) == 0
    torch.cuda.synchronize()
