"""What each layer's constructor puts in HBM (A25): sessions are built with
a seed and NO injected weights, and every parameter is read back and checked
against the distribution the reference's constructor draws from.

  Linear(in, out, ..., "xavier")   W U(+-sqrt(6/(in+out))), b 0     (linear.cpp:70-80, init.cpp:21-33)
  Conv2D(C, OC, k)                 W U(+-sqrt(6/(C k^2 + OC k^2))), b 0   (conv2d.cpp:42-56)
  LSTM(I, H)                       W_ih U(+-sqrt(6/(I+H))), W_hh U(+-sqrt(6/2H)),
                                   b 0 except the forget block [H, 2H) = 1  (lstm.cpp:42-51)
  GRU(I, H)                        same limits, b 0                   (gru.cpp:36-44)
  RNN(I, H)                        xavier [I,H], [H,H], b 0            (rnn.cpp:33-36)
  Embedding(V, D)                  U(+-1/sqrt(D)) on [V, D]           (embedding.cpp:38-39)
  MultiHeadAttention(D, h)         four xavier [D, D]                 (attention.cpp:47-50)
  BatchNorm(F)                     gamma 1, beta 0                    (batch_norm.cpp:25-40)

The limits of different layers differ by factors of 2-6 at these shapes
(e.g. a conv fan of C instead of C k^2 would give a 3x larger limit), so a
wrong fan or formula fails the support check (tests/init_stats.py).  Two
sessions with one seed hold identical parameters; another seed differs.
"""
import numpy as np
import pytest

from cppnet_amd import trainer
from init_stats import check_uniform

pytestmark = pytest.mark.gpu


def _params(cfg):
    s = trainer.Session(cfg)
    try:
        return s.get_params()
    finally:
        s.close()


def _u(w, L):
    check_uniform(np.asarray(w, np.float64), -L, L)


def test_linear_xavier_and_zero_bias(gpu):
    cfg = trainer.MLPConfig("init mlp", [96, 160, 40, 3], "relu", "none", "softmax_ce", 8, seed=11)
    p = _params(cfg)
    for li, (i, o) in enumerate(zip(cfg.sizes[:-1], cfg.sizes[1:])):
        W, b = p[2 * li], p[2 * li + 1]
        assert W.size == i * o and b.size == o
        _u(W, np.sqrt(6.0 / (i + o)))
        assert np.all(b == 0.0)


def test_conv_fans_include_kernel_area(gpu):
    cfg = trainer.CNNConfig("init cnn", [(3, 16, 3, 1, 1), (16, 24, 5, 1, 2)], 2, [2, 3, 16, 16], 10,
                            seed=12)
    p = _params(cfg)
    for ci, (ic, oc, k, _, _) in enumerate(cfg.convs):
        W, b = p[2 * ci], p[2 * ci + 1]
        assert W.size == oc * ic * k * k
        _u(W, np.sqrt(6.0 / (ic * k * k + oc * k * k)))
        assert np.all(b == 0.0)
    F = cfg.flat_features()
    _u(p[4], np.sqrt(6.0 / (F + 10)))
    assert np.all(p[5] == 0.0)


@pytest.mark.parametrize("cell", ["lstm", "gru", "rnn"])
def test_recurrent_limits_and_forget_bias(gpu, cell):
    I, H = 48, 64
    cfg = trainer.RNNConfig(f"init {cell}", cell, 4, 3, I, H, seed=13)
    p = _params(cfg)
    G = trainer.GATES[cell] * H
    W_ih, W_hh, b = p[0], p[1], p[2]
    assert W_ih.size == I * G and W_hh.size == H * G and b.size == G
    _u(W_ih, np.sqrt(6.0 / (I + H)))
    _u(W_hh, np.sqrt(6.0 / (2 * H)))
    want = np.zeros(G, np.float32)
    if cell == "lstm":
        want[H:2 * H] = 1.0  # gate order i, f, g, o: the forget block
    assert np.array_equal(b, want)
    _u(p[3], np.sqrt(6.0 / (H + 1)))
    assert np.all(p[4] == 0.0)


def test_embedding_attention_batchnorm(gpu):
    cfg = trainer.transformer_config(5, batch=2, seq_len=8, vocab=300, embed_dim=64, heads=4, blocks=1,
                                     ffn=128, classes=4)
    cfg.seed = 14
    p = _params(cfg)
    D, V, F = cfg.embed_dim, cfg.vocab, cfg.ffn
    assert p[0].size == V * D
    _u(p[0], 1.0 / np.sqrt(D))
    for i in range(4):  # W_q, W_k, W_v, W_o
        assert p[1 + i].size == D * D
        _u(p[1 + i], np.sqrt(6.0 / (2 * D)))
    assert np.all(p[5] == 1.0) and np.all(p[6] == 0.0)  # gamma, beta
    _u(p[7], np.sqrt(6.0 / (D + F)))
    assert np.all(p[8] == 0.0)
    _u(p[9], np.sqrt(6.0 / (F + D)))
    assert np.all(p[10] == 0.0)


def test_seed_reproducible(gpu):
    cfg = trainer.RNNConfig("init seed", "lstm", 4, 3, 16, 32, seed=21)
    a, b = _params(cfg), _params(cfg)
    assert all(np.array_equal(x, y) for x, y in zip(a, b))
    cfg.seed = 22
    c = _params(cfg)
    assert not np.array_equal(a[0], c[0]) and not np.array_equal(a[1], c[1])
