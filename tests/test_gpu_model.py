"""Model-level parity: the C++ trainer (CppNet-compatible classes on device
"gpu", libcppnet.so) against the oracle-composed model on identical seeded
inputs and injected weights (oracle/mlp.py).

Bars:
* one step: loss and every parameter gradient within rel 1e-4 / abs 1e-5
  (contractions magnitude-aware, see oracle_lib.close_mag), plus a ReLU-mask
  allowance: where a pre-activation lies within forward tolerance of 0, fp32
  rounding legitimately decides the mask either way, and the allowance is
  the most that choice can move each gradient (its own layer and, through
  dX, the layer below; _mask_allowance).  At most 1 in 10^4 entries of a
  tensor may need that allowance;
* updated weights after one step within the same bound, except where the
  reference gradient is itself within gradient tolerance of 0: Adam's first
  step moves W by ~lr*sign(g), so a sign that fp32 rounding cannot fix
  changes W by 2*lr.  Those elements are counted and must be that case;
* after many steps: every step's loss within rel 1e-3, and each parameter
  tensor within rel 1e-3 in norm -- or, where Adam's sign sensitivity makes
  the trajectory itself ill-conditioned, within twice the drift between two
  valid CPU evaluations of the same run (the oracle in fp32 and the oracle
  with double-accumulated contractions).  That drift is measured in the
  test and printed.
"""
import os

import numpy as np
import pytest

from cppnet_amd import trainer
from oracle.mlp import OracleMLP
from contraction_mags import rnn_mags, transformer_mags
from model_bars import _cnn_mags, _cnn_tie_allowance, _grad_mags, _mask_allowance
from oracle_lib import close, close_mag, fp, gemm_mag

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def oracle_mt(oracle):
    oracle.cnref_set_threads(min(16, os.cpu_count() or 1))
    return oracle


def _one_step(oracle, cfg, seed):
    rng = np.random.default_rng(seed)
    params, X, Y = trainer.synthetic_mlp(cfg, rng)
    sess = trainer.Session(cfg)
    sess.set_params(params)
    sess.set_batch(X, Y)
    ref = OracleMLP(cfg, oracle)
    ref.set_params(params)
    loss_gpu = sess.forward_backward()
    sess.grads_before_update = sess.get_grads()
    sess.update()
    loss_ref = ref.step(X, Y)
    return sess, ref, params, loss_gpu, loss_ref


@pytest.mark.parametrize("config,batch", [(1, None), (2, 256), (2, None)])
def test_one_step_parity(gpu, oracle_mt, config, batch):
    cfg = trainer.mlp_config(config, batch)
    print(f"[model] config {config} batch {cfg.batch}: one step", flush=True)
    _check_one_step(oracle_mt, cfg, 100 + config, f"config {config}")


# The reference's other activations, losses and optimizers in the same
# harness step (LeakyReLU, Softmax, CategoricalCrossEntropy, MAE, Huber, SGD,
# Momentum, Adagrad, RMSProp).
VARIANTS = [
    ("leaky_relu", "none", "cce", "sgd"),
    ("leaky_relu", "none", "cce", "momentum"),
    ("relu", "none", "huber", "adagrad"),
    ("tanh", "softmax", "mae", "rmsprop"),
    ("leaky_relu", "softmax", "mse", "adam"),
]


def _variant_cfg(hidden, out, loss, opt, batch=256):
    cfg = trainer.MLPConfig(f"MLP 48-96-64-10 {hidden}/{out} {loss} {opt}", [48, 96, 64, 10], hidden,
                            out, loss, batch, lr=1e-2 if opt in ("sgd", "momentum") else 1e-3)
    cfg.optimizer, cfg.opt_hyper, cfg.opt_eps = opt, 0.9, 1e-8
    return cfg


@pytest.mark.parametrize("hidden,out,loss,opt", VARIANTS)
def test_one_step_parity_variants(gpu, oracle_mt, hidden, out, loss, opt):
    cfg = _variant_cfg(hidden, out, loss, opt)
    print(f"[model] {cfg.name}: one step", flush=True)
    _check_one_step(oracle_mt, cfg, 7, cfg.name)


@pytest.mark.parametrize("hidden,out,loss,opt", VARIANTS[:4])
def test_multi_step_parity_variants(gpu, oracle_mt, hidden, out, loss, opt):
    cfg = _variant_cfg(hidden, out, loss, opt, batch=64)
    steps = 15
    print(f"[model] {cfg.name}: {steps} steps", flush=True)
    rng = np.random.default_rng(77)
    params, _, _ = trainer.synthetic_mlp(cfg, rng)
    sess = trainer.Session(cfg)
    sess.set_params(params)
    ref, ref_d = OracleMLP(cfg, oracle_mt), OracleMLP(cfg, oracle_mt)
    ref.set_params(params)
    ref_d.set_params(params)
    for step in range(steps):
        _, X, Y = trainer.synthetic_mlp(cfg, rng)
        sess.set_batch(X, Y)
        lg, lr_ = sess.step(), ref.step(X, Y)
        oracle_mt.cnref_set_accumulate_double(1)
        try:
            ref_d.step(X, Y)
        finally:
            oracle_mt.cnref_set_accumulate_double(0)
        assert abs(lg - lr_) <= 1e-3 * abs(lr_) + 1e-6, f"step {step}: loss {lg} vs {lr_}"
    for k, (a, b, c) in enumerate(zip(sess.get_params(), ref.get_params(), ref_d.get_params())):
        rel, drift = _rel(a, b), _rel(c, b)
        assert rel <= max(1e-3, 2.0 * drift), f"param {k}: relative norm error {rel:.3g}"
    sess.close()


def test_set_optimizer_refused_after_update(gpu):
    cfg = _variant_cfg("relu", "none", "mse", "adam", batch=8)
    params, X, Y = trainer.synthetic_mlp(cfg, np.random.default_rng(3))
    sess = trainer.Session(cfg)
    sess.set_batch(X, Y)
    sess.step()
    lib = trainer.load()
    assert lib.cnt_set_optimizer(sess.h, trainer.OPT["sgd"], 0.0, 0.0) != 0
    assert "already updated" in lib.cnt_last_error().decode()
    sess.close()


def _check_one_step(oracle_mt, cfg, seed, label):
    config = label
    sess, ref, params, loss_gpu, loss_ref = _one_step(oracle_mt, cfg, seed=seed)
    ok, msg = close([loss_gpu], [loss_ref], 1e-4, 1e-5)
    assert ok, f"loss: {msg}"
    mags = _grad_mags(oracle_mt, ref, cfg)
    allow = _mask_allowance(oracle_mt, ref, cfg, params)
    g_gpu = sess.grads_before_update
    n_allow = 0
    for k, (a, b, mag, al) in enumerate(zip(g_gpu, ref.last_grads, mags, allow)):
        ok, msg = close_mag(a, b, mag, 1e-4, 1e-5)
        if not ok:
            lim = 1e-5 + 1e-4 * np.maximum(np.abs(b), mag) + al
            err = np.abs(a.astype(np.float64) - b)
            bad = err > lim
            assert not bad.any(), (f"grad of param {k}: {int(bad.sum())} outside tolerance + "
                                   f"mask allowance ({msg})")
            needed = int((err > 1e-5 + 1e-4 * np.maximum(np.abs(b), mag)).sum())
            # the allowance is a loose upper bound: it may only rescue a handful of entries
            assert needed <= max(1, a.size // 10000), (
                f"grad of param {k}: {needed} entries needed the mask allowance ({msg})")
            n_allow += needed
    w_gpu = sess.get_params()
    flips = 0
    for k, (a, b, g, mag, al) in enumerate(zip(w_gpu, ref.get_params(), ref.last_grads, mags,
                                               allow)):
        err = np.abs(a.astype(np.float64) - b)
        lim = 1e-5 + 1e-4 * np.abs(b)
        bad = err > lim
        g_tol = 1e-5 + 1e-4 * np.maximum(np.abs(g), mag) + al
        unexplained = bad & (np.abs(g) > g_tol)
        assert not unexplained.any(), (
            f"param {k}: {int(unexplained.sum())} weights differ where the gradient is well "
            f"conditioned (max err {err[unexplained].max():.3g})")
        flips += int(bad.sum())
    total = sum(p.size for p in w_gpu)
    print(f"[model] {config}: loss {loss_gpu:.7f} vs {loss_ref:.7f}; {n_allow} grads "
          f"needed the ReLU-mask allowance; {flips}/{total} updated weights differ, all at |g| "
          f"within gradient tolerance of 0")
    sess.close()


def _check_grads_and_update(grads, ref, mags, updated):
    """Gradients within 1e-5 + 1e-4 max(|ref|, mag) elementwise; updated
    weights within 1e-5 + 1e-4 |ref| except where the gradient itself lies
    within its bar of 0 (Adam's first step is ~ -lr sign(g), so a sign that
    rounding decides moves the weight by up to 2 lr)."""
    for k, (a, b, m) in enumerate(zip(grads, ref.last_grads, mags)):
        ok, msg = close_mag(a, b, m, 1e-4, 1e-5)
        assert ok, f"grad of param {k}: {msg}"
    for k, (a, b, g, m) in enumerate(zip(updated, ref.get_params(), ref.last_grads, mags)):
        bad = np.abs(a.astype(np.float64) - b) > 1e-5 + 1e-4 * np.abs(b)
        ill = np.abs(g) <= 1e-5 + 1e-4 * np.maximum(np.abs(g), m)
        assert not (bad & ~ill).any(), (
            f"param {k}: {int((bad & ~ill).sum())} updated weights differ where the gradient is well "
            f"conditioned")


def _rel(a, b):
    return float(np.linalg.norm(a.astype(np.float64) - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("config,batch,steps", [(1, None, 100), (2, 128, 20)])
def test_multi_step_parity(gpu, oracle_mt, config, batch, steps):
    cfg = trainer.mlp_config(config, batch)
    print(f"[model] config {config} batch {cfg.batch}: {steps} steps", flush=True)
    rng = np.random.default_rng(7 + config)
    params, _, _ = trainer.synthetic_mlp(cfg, rng)
    batches = [trainer.synthetic_mlp(cfg, rng)[1:] for _ in range(steps)]
    sess = trainer.Session(cfg)
    sess.set_params(params)
    ref = OracleMLP(cfg, oracle_mt)
    ref.set_params(params)
    ref_d = OracleMLP(cfg, oracle_mt)  # same run, double-accumulated contractions
    ref_d.set_params(params)
    for step, (X, Y) in enumerate(batches):
        # a fresh batch each step, as a data loader would provide
        sess.set_batch(X, Y)
        lg, lr_ = sess.step(), ref.step(X, Y)
        oracle_mt.cnref_set_accumulate_double(1)
        try:
            ref_d.step(X, Y)
        finally:
            oracle_mt.cnref_set_accumulate_double(0)
        assert abs(lg - lr_) <= 1e-3 * abs(lr_) + 1e-6, f"step {step}: loss {lg} vs {lr_}"
    for k, (a, b, c) in enumerate(zip(sess.get_params(), ref.get_params(), ref_d.get_params())):
        rel, drift = _rel(a, b), _rel(c, b)
        print(f"[model] config {config} param {k}: gpu-vs-oracle {rel:.3g}, oracle fp32-vs-fp64acc "
              f"{drift:.3g} after {steps} steps")
        assert rel <= max(1e-3, 2.0 * drift), (
            f"param {k}: relative norm error {rel:.3g} after {steps} steps "
            f"(oracle's own rounding drift {drift:.3g})")
    sess.close()


def test_loss_reaches_device_without_sync_until_read(gpu):
    cfg = trainer.mlp_config(1, 64)
    params, X, Y = trainer.synthetic_mlp(cfg, np.random.default_rng(0))
    sess = trainer.Session(cfg)
    sess.set_params(params)
    sess.set_batch(X, Y)
    for _ in range(5):
        assert sess.step(read_loss=False) is None
    loss = sess.step()
    assert np.isfinite(loss) and loss > 0
    sess.close()


def test_cnn_one_step_parity(gpu, oracle_mt):
    """Config 3 at full size (batch 256): loss and all six gradients."""
    from oracle.cnn import OracleCNN
    cfg = trainer.cnn_config(3)
    print(f"[model] config 3 batch {cfg.batch}: one step", flush=True)
    params, X, Y = trainer.synthetic_cnn(cfg, np.random.default_rng(303))
    sess = trainer.Session(cfg)
    sess.set_params(params)
    sess.set_batch(X, Y)
    ref = OracleCNN(cfg, oracle_mt)
    ref.set_params(params)
    loss_gpu = sess.forward_backward()
    grads = sess.get_grads()
    sess.update()
    after = sess.get_grads()
    # Conv2D::step clears its grads after the update (conv2d.cpp:211-212);
    # Linear::step does not (linear.cpp:126-146)
    assert all(not g.any() for g in after[:4]), "conv grads must be cleared by step()"
    np.testing.assert_array_equal(after[4], grads[4])
    loss_ref = ref.step(X, Y)
    ok, msg = close([loss_gpu], [loss_ref], 1e-4, 1e-5)
    assert ok, f"loss: {msg}"
    mags = _cnn_mags(oracle_mt, ref, cfg)
    allow = _cnn_tie_allowance(oracle_mt, ref, cfg, params)
    n_allow = 0
    for k, (a, b, mag, al) in enumerate(zip(grads, ref.last_grads, mags, allow)):
        ok, msg = close_mag(a, b, mag, 1e-4, 1e-5)
        if not ok:
            err = np.abs(a.astype(np.float64) - b)
            strict = 1e-5 + 1e-4 * np.maximum(np.abs(b), mag)
            bad = err > strict + (al if al.size == a.size else 0.0)
            assert not bad.any(), f"grad of param {k}: {int(bad.sum())} beyond tolerance + tie allowance ({msg})"
            needed = int((err > strict).sum())
            # the allowance is an upper bound on routing flips: it may rescue at most 1 in 10^3
            assert needed <= max(1, a.size // 1000), f"grad of param {k}: {needed} needed the tie allowance"
            n_allow += needed
    print(f"[model] config 3: loss {loss_gpu:.7f} vs {loss_ref:.7f}; {n_allow} grads needed the "
          "ReLU/max-pool tie allowance")
    sess.close()


def test_cnn_multi_step_parity(gpu, oracle_mt):
    from oracle.cnn import OracleCNN
    cfg = trainer.cnn_config(3, batch=16)
    steps = 8
    print(f"[model] config 3 batch {cfg.batch}: {steps} steps", flush=True)
    rng = np.random.default_rng(31)
    params, _, _ = trainer.synthetic_cnn(cfg, rng)
    sess = trainer.Session(cfg)
    sess.set_params(params)
    ref, ref_d = OracleCNN(cfg, oracle_mt), OracleCNN(cfg, oracle_mt)
    ref.set_params(params)
    ref_d.set_params(params)
    for step in range(steps):
        _, X, Y = trainer.synthetic_cnn(cfg, rng)
        sess.set_batch(X, Y)
        lg, lr_ = sess.step(), ref.step(X, Y)
        oracle_mt.cnref_set_accumulate_double(1)
        try:
            ref_d.step(X, Y)
        finally:
            oracle_mt.cnref_set_accumulate_double(0)
        assert abs(lg - lr_) <= 1e-3 * abs(lr_) + 1e-6, f"step {step}: loss {lg} vs {lr_}"
    for k, (a, b, c) in enumerate(zip(sess.get_params(), ref.get_params(), ref_d.get_params())):
        rel, drift = _rel(a, b), _rel(c, b)
        print(f"[model] config 3 param {k}: gpu-vs-oracle {rel:.3g}, oracle drift {drift:.3g}")
        assert rel <= max(1e-3, 2.0 * drift), f"param {k}: relative norm error {rel:.3g}"
    sess.close()


@pytest.mark.parametrize("cell,batch,seq", [("lstm", None, None), ("gru", 32, 16), ("rnn", 32, 16)])
def test_rnn_one_step_parity(gpu, oracle_mt, cell, batch, seq):
    """Config 4 (LSTM 128->512, T=64, batch 128) at full size, and the GRU
    and Elman variants of the same regressor.  The recurrent grads are sums
    over all B*S timestep-rows; each element's relative bound is taken
    against max(|ref|, (|A|^T |dpre|)/sqrt(B*S)) with A its contraction's
    other operand (x_t, h_{t-1} or r*h_{t-1}) and dpre the oracle's gate
    pre-activation gradients (tests/contraction_mags.py)."""
    from oracle.rnn import OracleSeqRegressor
    cfg = trainer.rnn_config(4, batch=batch, seq_len=seq, cell=cell)
    print(f"[model] config 4 {cell} batch {cfg.batch} T={cfg.seq_len}: one step", flush=True)
    params, X, Y = trainer.synthetic_rnn(cfg, np.random.default_rng(404))
    sess = trainer.Session(cfg)
    sess.set_params(params)
    sess.set_batch(X, Y)
    ref = OracleSeqRegressor(cfg, oracle_mt)
    ref.set_params(params)
    loss_gpu = sess.forward_backward()
    grads = sess.get_grads()
    sess.update()
    after = sess.get_grads()
    assert all(not g.any() for g in after[:3]), "recurrent grads must be cleared by step()"
    loss_ref = ref.step(X, Y)
    ok, msg = close([loss_gpu], [loss_ref], 1e-4, 1e-5)
    assert ok, f"loss: {msg}"
    mags = rnn_mags(oracle_mt, ref, cfg)
    _check_grads_and_update(grads, ref, mags, sess.get_params())
    print(f"[model] config 4 {cell}: loss {loss_gpu:.7f} vs {loss_ref:.7f}")
    sess.close()


@pytest.mark.parametrize("cell,opt", [("lstm", "adam"), ("rnn", "momentum"), ("gru", "rmsprop")])
def test_rnn_multi_step_parity(gpu, oracle_mt, cell, opt):
    from oracle.rnn import OracleSeqRegressor
    cfg = trainer.rnn_config(4, batch=16, seq_len=12, cell=cell)
    cfg.optimizer = opt
    steps = 20
    print(f"[model] config 4 {cell} {opt} batch {cfg.batch} T={cfg.seq_len}: {steps} steps", flush=True)
    rng = np.random.default_rng(41)
    params, _, _ = trainer.synthetic_rnn(cfg, rng)
    sess = trainer.Session(cfg)
    sess.set_params(params)
    ref, ref_d = OracleSeqRegressor(cfg, oracle_mt), OracleSeqRegressor(cfg, oracle_mt)
    ref.set_params(params)
    ref_d.set_params(params)
    for step in range(steps):
        _, X, Y = trainer.synthetic_rnn(cfg, rng)
        sess.set_batch(X, Y)
        lg, lr_ = sess.step(), ref.step(X, Y)
        oracle_mt.cnref_set_accumulate_double(1)
        try:
            ref_d.step(X, Y)
        finally:
            oracle_mt.cnref_set_accumulate_double(0)
        assert abs(lg - lr_) <= 1e-3 * abs(lr_) + 1e-6, f"step {step}: loss {lg} vs {lr_}"
    for k, (a, b, c) in enumerate(zip(sess.get_params(), ref.get_params(), ref_d.get_params())):
        rel, drift = _rel(a, b), _rel(c, b)
        print(f"[model] config 4 param {k}: gpu-vs-oracle {rel:.3g}, oracle drift {drift:.3g}")
        assert rel <= max(1e-3, 2.0 * drift), f"param {k}: relative norm error {rel:.3g}"
    sess.close()


def test_transformer_one_step_parity(gpu, oracle_mt):
    """Config 5 at full size (Embedding 8192x512, 2 encoder blocks, B=32,
    S=256): loss, every gradient (relative part against max(|ref|, the
    per-element magnitude (|A|^T|B|)/sqrt(R) of its contraction over the
    R = 8192 rows, tests/contraction_mags.py) and the updated weights; the
    embedding gradient's routing is exact (rows of ids absent from the batch
    stay exactly 0)."""
    from oracle.transformer import OracleTransformer
    cfg = trainer.transformer_config(5)
    print(f"[model] config 5 batch {cfg.batch} S={cfg.seq_len}: one step", flush=True)
    params, ids, Y = trainer.synthetic_transformer(cfg, np.random.default_rng(505))
    sess = trainer.Session(cfg)
    sess.set_params(params)
    np.testing.assert_array_equal(sess.get_params()[0], params[0])  # layout round trip
    sess.set_batch(ids, Y)
    ref = OracleTransformer(cfg, oracle_mt)
    ref.set_params(params)
    loss_gpu = sess.forward_backward()
    grads = sess.get_grads()
    sess.update()
    after = sess.get_grads()
    n_lin = {len(params) - 2, len(params) - 1} | {1 + 10 * i + j for i in range(cfg.blocks) for j in (6, 7, 8, 9)}
    assert all(not g.any() for k, g in enumerate(after) if k not in n_lin), \
        "Embedding / MHA / BatchNorm grads must be cleared by step()"
    loss_ref = ref.step(ids, Y)
    ok, msg = close([loss_gpu], [loss_ref], 1e-4, 1e-5)
    assert ok, f"loss: {msg}"
    absent = np.setdiff1d(np.arange(cfg.vocab), ids)
    emb_g = grads[0].reshape(cfg.embed_dim, cfg.vocab)  # ColMajor [V, D]: column d
    assert not emb_g[:, absent].any(), "embedding rows of absent ids must stay exactly 0"
    assert np.all(emb_g[:, np.unique(ids)].any(axis=0))
    mags = transformer_mags(oracle_mt, ref, cfg)
    _check_grads_and_update(grads, ref, mags, sess.get_params())
    print(f"[model] config 5: loss {loss_gpu:.7f} vs {loss_ref:.7f}")
    sess.close()


def test_transformer_multi_step_parity(gpu, oracle_mt):
    from oracle.transformer import OracleTransformer
    cfg = trainer.transformer_config(5, batch=4, seq_len=16, vocab=64, embed_dim=32, heads=4, blocks=2,
                                     ffn=64, classes=4)
    steps = 20
    print(f"[model] config 5 (reduced) {steps} steps", flush=True)
    rng = np.random.default_rng(55)
    params, _, _ = trainer.synthetic_transformer(cfg, rng)
    sess = trainer.Session(cfg)
    sess.set_params(params)
    ref, ref_d = OracleTransformer(cfg, oracle_mt), OracleTransformer(cfg, oracle_mt)
    ref.set_params(params)
    ref_d.set_params(params)
    for step in range(steps):
        _, ids, Y = trainer.synthetic_transformer(cfg, rng)
        sess.set_batch(ids, Y)
        lg, lr_ = sess.step(), ref.step(ids, Y)
        oracle_mt.cnref_set_accumulate_double(1)
        try:
            ref_d.step(ids, Y)
        finally:
            oracle_mt.cnref_set_accumulate_double(0)
        assert abs(lg - lr_) <= 1e-3 * abs(lr_) + 1e-6, f"step {step}: loss {lg} vs {lr_}"
    for k, (a, b, c) in enumerate(zip(sess.get_params(), ref.get_params(), ref_d.get_params())):
        rel, drift = _rel(a, b), _rel(c, b)
        print(f"[model] config 5 param {k}: gpu-vs-oracle {rel:.3g}, oracle drift {drift:.3g}")
        assert rel <= max(1e-3, 2.0 * drift), f"param {k}: relative norm error {rel:.3g}"
    sess.close()


def test_transformer_rejects_out_of_range_ids(gpu):
    cfg = trainer.transformer_config(5, batch=2, seq_len=3, vocab=10, embed_dim=8, heads=2, blocks=1,
                                     ffn=16, classes=2)
    params, ids, Y = trainer.synthetic_transformer(cfg, np.random.default_rng(1))
    sess = trainer.Session(cfg)
    ids = ids.copy()
    ids[4] = 10
    # the trainer checks ids when the batch is uploaded, with the reference's
    # message (embedding.cpp:87-90), so the steps never read back
    with pytest.raises(Exception, match="token ID 10 out of range"):
        sess.set_batch(ids, Y)
    ids[4] = -1
    with pytest.raises(Exception, match="token ID -1 out of range"):
        sess.set_batch(ids, Y)
    ids[4] = 9
    sess.set_batch(ids, Y)
    assert np.isfinite(sess.step())
    sess.close()
