"""Per-element error-bar magnitudes of the recurrent (config 4) and
transformer (config 5) parameter gradients, from the oracle's traced
operands (oracle/rnn.py, oracle/transformer.py; the traces themselves are
pinned in tests/test_oracle_traces.py).

Every such gradient is a contraction G = A^T B over R rows (the B*S
timestep-rows of a sequence, or the samples of a batch); rounding a length-R
fp32 sum that partly cancels leaves about u*sqrt(R) of (|A|^T |B|)/sqrt(R) on
any evaluation order, so that is the magnitude the relative bar is taken
against (as for the MLP and CNN gradients).  Biases and BatchNorm's
gamma/beta use the same with A = 1 or A = xhat; the embedding table's rows
sum the gradient rows of each token's positions.

Each function returns one magnitude array per parameter, in session order,
each laid out like the parameter (ColMajor)."""
from __future__ import annotations

import numpy as np

from oracle_lib import gemm_mag


def _shift_rows(Y, R, B, H):
    """[R, H] ColMajor rows r -> rows r - B (zero for the first B): h_{t-1}."""
    y = Y.reshape(H, R)
    out = np.zeros_like(y)
    out[:, B:] = y[:, :R - B]
    return out.ravel()


def rnn_mags(oracle, ref, cfg):
    B, S, I, H, O = cfg.batch, cfg.seq_len, cfg.input_size, cfg.hidden, cfg.out_features
    R = B * S
    tr = ref.trace
    dpre = tr["dpre"]
    G = dpre.size // R
    Hp = _shift_rows(tr["Yseq"], R, B, H)
    m_ih = gemm_mag(oracle, 1, 0, I, G, R, tr["X"], R, dpre, R, I)
    if cfg.cell == "gru":  # z, r blocks against h_{t-1}; the n block against r*h_{t-1}
        zr = gemm_mag(oracle, 1, 0, H, 2 * H, R, Hp, R, dpre, R, H)
        n = gemm_mag(oracle, 1, 0, H, H, R, tr["rh"], R, dpre[2 * H * R:], R, H)
        m_hh = np.concatenate([zr, n])
    else:
        m_hh = gemm_mag(oracle, 1, 0, H, G, R, Hp, R, dpre, R, H)
    m_b = gemm_mag(oracle, 1, 0, 1, G, R, np.ones(R, np.float32), R, dpre, R, 1)
    m_w = gemm_mag(oracle, 1, 0, H, O, B, tr["hT"], B, tr["g"], B, H)
    m_bb = gemm_mag(oracle, 1, 0, 1, O, B, np.ones(B, np.float32), B, tr["g"], B, 1)
    return [m_ih, m_hh, m_b, m_w, m_bb]


def _demb_mag(oracle, ref, cfg, params):
    """Per-element size of the gradient reaching the embedding, dy = dX_attn +
    dr of the first block (oracle/transformer.py): the attention input
    gradient is a contraction over the 3D columns of [gQp gKp gVp] with
    [Wq Wk Wv]^T, and BatchNorm's dr = gamma/sigma (gh - mean(gh) - xhat
    mean(gh xhat)) with gh = dy + dz1 W1^T, itself a contraction over F.
    Each contraction contributes (|A||B|)/sqrt(K), the other terms their
    absolute values; ColMajor [R, D]."""
    B, S, D, F = cfg.batch, cfg.seq_len, cfg.embed_dim, cfg.ffn
    R = B * S
    T = ref.trace[0]
    Wq, Wk, Wv, _, gam, _, W1 = (params[j] for j in range(1, 8))
    dxa = sum(gemm_mag(oracle, 0, 1, R, D, D, T[g], R, W, D, R) for g, W in (("gQp", Wq), ("gKp", Wk), ("gVp", Wv)))
    dxa /= np.float32(np.sqrt(3.0))  # three sums over D each: one over 3D
    gh_mag = np.abs(T["gh"]) + gemm_mag(oracle, 0, 1, R, D, F, T["dz1"], R, W1, D, R)
    gh, xh = T["gh"].reshape(D, R), T["xh"].reshape(D, R)
    inv_sigma = 1.0 / np.sqrt(T["bv"].astype(np.float64) + 1e-5)
    scale = (np.abs(gam) * inv_sigma)[:, None]
    dr = scale * (gh_mag.reshape(D, R) + np.abs(gh.mean(axis=1))[:, None]
                  + np.abs(xh) * np.abs((gh * xh).mean(axis=1))[:, None])
    return (np.abs(ref.head_trace["demb"]) + dxa + dr.ravel()).astype(np.float32)


def transformer_mags(oracle, ref, cfg, params=None):
    """params: the weights the step's backward used (default: the oracle's
    current ones, i.e. after its update, close enough for a magnitude)."""
    B, S, V, D, F, C = cfg.batch, cfg.seq_len, cfg.vocab, cfg.embed_dim, cfg.ffn, cfg.classes
    R = B * S
    ones = np.ones(R, np.float32)
    ht = ref.head_trace
    # embedding rows: the sum over each token's positions of the size of the
    # gradient reaching the embedding, / sqrt(count)
    ids = ht["ids"].astype(np.int64)
    demb = _demb_mag(oracle, ref, cfg, ref.params if params is None else params).reshape(D, R)
    acc = np.zeros((D, V), np.float64)
    np.add.at(acc.T, ids, demb.T)
    cnt = np.bincount(ids, minlength=V).astype(np.float64)
    emb = (acc / np.sqrt(np.maximum(cnt, 1.0))).T  # [V, D] logical
    mags = [np.ascontiguousarray(emb.T).ravel().astype(np.float32)]  # ColMajor [V, D]
    for T in ref.trace:
        x = T["x"]
        mags += [gemm_mag(oracle, 1, 0, D, D, R, x, R, T["gQp"], R, D),
                 gemm_mag(oracle, 1, 0, D, D, R, x, R, T["gKp"], R, D),
                 gemm_mag(oracle, 1, 0, D, D, R, x, R, T["gVp"], R, D),
                 gemm_mag(oracle, 1, 0, D, D, R, T["ctx"], R, T["dr"], R, D)]
        # BatchNorm: dgamma = sum_rows gh * xhat, dbeta = sum_rows gh
        xh, gh = T["xh"].reshape(D, R), T["gh"].reshape(D, R)
        mags += [(np.abs(xh * gh).sum(axis=1) / np.sqrt(R)).astype(np.float32),
                 (np.abs(gh).sum(axis=1) / np.sqrt(R)).astype(np.float32)]
        mags += [gemm_mag(oracle, 1, 0, D, F, R, T["h"], R, T["dz1"], R, D),
                 gemm_mag(oracle, 1, 0, 1, F, R, ones, R, T["dz1"], R, 1),
                 gemm_mag(oracle, 1, 0, F, D, R, T["g1"], R, T["dy"], R, F),
                 gemm_mag(oracle, 1, 0, 1, D, R, ones, R, T["dy"], R, 1)]
    mags += [gemm_mag(oracle, 1, 0, D, C, B, ht["pooled"], B, ht["gl"], B, D),
             gemm_mag(oracle, 1, 0, 1, C, B, np.ones(B, np.float32), B, ht["gl"], B, 1)]
    return mags
