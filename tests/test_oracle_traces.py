"""Pins the oracle's traced operands (CPU only).  The GPU parity tests build
their per-element error bars from these traces (tests/contraction_mags.py),
so each trace must be the true operand of its gradient contraction: every
weight gradient the oracle returns must equal, to float64 rounding of fp32
sums, the contraction of the traced operands (e.g. gW_ih = X^T dpre over all
B*S timestep-rows, gW_q = x^T gQp, dgamma = sum(gh * xhat))."""
import numpy as np
import pytest

from cppnet_amd import trainer
from oracle.rnn import OracleSeqRegressor
from oracle.transformer import OracleTransformer


def cm(flat, rows, cols):
    return np.asarray(flat, np.float64).reshape(cols, rows).T


def close(got, want, what):
    scale = np.abs(want).max() + 1e-30
    err = np.abs(np.asarray(got, np.float64) - want).max() / scale
    assert err < 1e-5, f"{what}: max rel err {err:.3g}"


@pytest.mark.parametrize("cell", ["lstm", "gru", "rnn"])
def test_recurrent_dpre_trace(oracle, cell):
    cfg = trainer.rnn_config(4, batch=5, seq_len=4, cell=cell)
    cfg.input_size, cfg.hidden = 6, 7
    params, X, Y = trainer.synthetic_rnn(cfg, np.random.default_rng(8))
    ref = OracleSeqRegressor(cfg, oracle)
    ref.set_params(params)
    ref.step(X, Y)
    B, S, I, H = cfg.batch, cfg.seq_len, cfg.input_size, cfg.hidden
    R = B * S
    G = trainer.GATES[cell] * H
    tr = ref.trace
    dpre, Xm, Ym = cm(tr["dpre"], R, G), cm(tr["X"], R, I), cm(tr["Yseq"], R, H)
    Hp = np.zeros_like(Ym)
    Hp[B:] = Ym[:R - B]  # row n + B t holds h_{t-1}
    close(ref.last_grads[0], (Xm.T @ dpre).T.ravel(), "gW_ih")
    if cell == "gru":
        want = np.concatenate([Hp.T @ dpre[:, :2 * H], cm(tr["rh"], R, H).T @ dpre[:, 2 * H:]], axis=1)
    else:
        want = Hp.T @ dpre
    close(ref.last_grads[1], want.T.ravel(), "gW_hh")
    close(ref.last_grads[2], dpre.sum(axis=0), "gb")


def test_transformer_traces(oracle):
    cfg = trainer.transformer_config(5, batch=3, seq_len=5, vocab=20, embed_dim=8, heads=2, blocks=2, ffn=12,
                                     classes=3)
    params, ids, Y = trainer.synthetic_transformer(cfg, np.random.default_rng(9))
    ref = OracleTransformer(cfg, oracle)
    ref.set_params(params)
    ref.step(ids, Y)
    R, D, F = cfg.batch * cfg.seq_len, cfg.embed_dim, cfg.ffn
    g = ref.last_grads
    for i, T in enumerate(ref.trace):
        base = 1 + 10 * i
        x = cm(T["x"], R, D)
        close(g[base + 0], (x.T @ cm(T["gQp"], R, D)).T.ravel(), f"block {i} gW_q")
        close(g[base + 1], (x.T @ cm(T["gKp"], R, D)).T.ravel(), f"block {i} gW_k")
        close(g[base + 2], (x.T @ cm(T["gVp"], R, D)).T.ravel(), f"block {i} gW_v")
        close(g[base + 3], (cm(T["ctx"], R, D).T @ cm(T["dr"], R, D)).T.ravel(), f"block {i} gW_o")
        gh, xh = cm(T["gh"], R, D), cm(T["xh"], R, D)
        close(g[base + 4], (gh * xh).sum(axis=0), f"block {i} dgamma")
        close(g[base + 5], gh.sum(axis=0), f"block {i} dbeta")
        close(g[base + 6], (cm(T["h"], R, D).T @ cm(T["dz1"], R, F)).T.ravel(), f"block {i} gW_1")
        close(g[base + 8], (cm(T["g1"], R, F).T @ cm(T["dy"], R, D)).T.ravel(), f"block {i} gW_2")
    ht = ref.head_trace
    B, C = cfg.batch, cfg.classes
    close(g[-2], (cm(ht["pooled"], B, D).T @ cm(ht["gl"], B, C)).T.ravel(), "classifier W")
    # embedding rows: the sum of each token's positions' gradient rows ([V, D] ColMajor)
    demb, want = cm(ht["demb"], R, D), np.zeros((cfg.vocab, D))
    np.add.at(want, ht["ids"].astype(np.int64), demb)
    close(g[0], want.T.ravel(), "embedding")


@pytest.mark.parametrize("cell", ["lstm", "gru", "rnn"])
def test_rnn_mags_layout(oracle, cell):
    from contraction_mags import rnn_mags
    cfg = trainer.rnn_config(4, batch=4, seq_len=3, cell=cell)
    cfg.input_size, cfg.hidden = 5, 6
    params, X, Y = trainer.synthetic_rnn(cfg, np.random.default_rng(2))
    ref = OracleSeqRegressor(cfg, oracle)
    ref.set_params(params)
    ref.step(X, Y)
    mags = rnn_mags(oracle, ref, cfg)
    assert [m.size for m in mags] == [p.size for p in params]
    for m, gr in zip(mags, ref.last_grads):
        # |sum| <= sum |.| = sqrt(R) * magnitude: the bar never undercuts the value
        assert np.all(np.abs(gr) <= np.sqrt(cfg.batch * cfg.seq_len) * m * (1 + 1e-5) + 1e-12)


def test_transformer_mags_layout(oracle):
    from contraction_mags import transformer_mags
    cfg = trainer.transformer_config(5, batch=2, seq_len=4, vocab=16, embed_dim=8, heads=2, blocks=1, ffn=12,
                                     classes=3)
    params, ids, Y = trainer.synthetic_transformer(cfg, np.random.default_rng(3))
    ref = OracleTransformer(cfg, oracle)
    ref.set_params(params)
    ref.step(ids, Y)
    mags = transformer_mags(oracle, ref, cfg)
    assert [m.size for m in mags] == [p.size for p in params]
    R = cfg.batch * cfg.seq_len
    for k, (m, gr) in enumerate(zip(mags, ref.last_grads)):
        assert np.all(np.abs(gr) <= np.sqrt(R) * m * (1 + 1e-5) + 1e-12), f"param {k}"


def test_sum_orders(oracle):
    """The oracle GEMM's alternative evaluation orders (used to measure how
    far a training trajectory moves under rounding alone) are what they say:
    each equals the sequential fp32 sum in its order, exactly."""
    from oracle import fp
    rng = np.random.default_rng(5)
    K = 300
    a = (rng.standard_normal(K) * np.logspace(0, 6, K)).astype(np.float32)
    b = np.ones(K, np.float32)

    def run(order):
        oracle.cnref_set_sum_order(order)
        c = np.zeros(1, np.float32)
        try:
            oracle.cnref_gemm_f32(0, 0, 1, 1, K, 1.0, fp(a), 1, fp(b), K, 0.0, fp(c), 1, None, 0)
        finally:
            oracle.cnref_set_sum_order(0)
        return c[0]

    def seq(xs):
        s = np.float32(0)
        for x in xs:
            s = np.float32(s + x)
        return s

    chunked = np.float32(0)
    for c0 in range(0, K, 32):
        chunked = np.float32(chunked + seq(a[c0:c0 + 32]))

    def tree(xs):  # 8 strided partial sums, combined pairwise
        q = [seq(xs[p::8]) for p in range(8)]
        return np.float32(np.float32(np.float32(q[0] + q[1]) + np.float32(q[2] + q[3])) +
                          np.float32(np.float32(q[4] + q[5]) + np.float32(q[6] + q[7])))

    # the GEMM applies order 3 per k-panel of 256, the panels added in turn
    strided = np.float32(tree(a[:256]) + tree(a[256:]))
    assert run(0) == seq(a)
    assert run(1) == seq(a[::-1])
    assert run(2) == chunked
    assert run(3) == strided
    assert len({float(run(o)) for o in range(4)}) == 4  # the orders differ on this input
    # the column sums (bias gradients) follow the same orders, order 3 over the whole column
    for order, want in ((0, seq(a)), (1, seq(a[::-1])), (2, chunked), (3, tree(a))):
        oracle.cnref_set_sum_order(order)
        out = np.zeros(1, np.float32)
        try:
            oracle.cnref_column_sum(fp(a), fp(out), K, 1, 0)
        finally:
            oracle.cnref_set_sum_order(0)
        assert out[0] == want, f"column sum, order {order}"
