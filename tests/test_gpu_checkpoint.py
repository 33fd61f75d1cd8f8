"""Model files of training sessions (Utils::save_model / load_model /
save_checkpoint / load_checkpoint through cnt_*).

* The CNET file is the reference's format (serialization.cpp:143-256): a
  parser written here from that format reads back exactly the session's
  parameters in the reference's layout, and a file built here from that
  format loads into a session exactly.
* A checkpoint starts with the same bytes as the CNET file, so the
  reference's reader loads it, and resumes exactly: a fresh session with
  other initial weights that loads it continues bit for bit as the saved
  session does, optimizer state and step counts included.
"""
import struct

import numpy as np
import pytest

from cppnet_amd import trainer

pytestmark = pytest.mark.gpu

MAGIC = 0x434E4554


def _record(buf, off):
    nd = struct.unpack_from("<i", buf, off)[0]
    dims = list(struct.unpack_from(f"<{nd}i", buf, off + 4))
    off += 4 + 4 * nd
    n = int(np.prod(dims)) if dims else 1
    data = np.frombuffer(buf, np.float32, n, off).copy()
    return dims, data, off + 4 * n


def _parse_cnet(buf):
    magic, nlayers = struct.unpack_from("<ii", buf, 0)
    assert magic == MAGIC
    off, recs = 8, []
    while off < len(buf) and len(recs) < nlayers:
        t = struct.unpack_from("<i", buf, off)[0]
        if t == 0x434E5831:  # the checkpoint extension begins
            break
        off += 4
        n_tensors = {0: 0, 1: 2, 2: 4, 3: 1}[t]
        tensors = []
        for _ in range(n_tensors):
            if t == 1 and len(tensors) == 1 and struct.unpack_from("<i", buf, off)[0] != 1:
                break  # a Linear without bias
            dims, data, off = _record(buf, off)
            tensors.append((dims, data))
        recs.append((t, tensors))
    return nlayers, recs, off


def _put(dims, data):
    return struct.pack(f"<i{len(dims)}i", len(dims), *dims) + np.asarray(data, np.float32).tobytes()


def _mlp_cfg(opt="adam"):
    cfg = trainer.MLPConfig("MLP 20-32-16-3", [20, 32, 16, 3], "relu", "none", "softmax_ce", 24)
    cfg.optimizer = opt
    return cfg


def _tf_cfg():
    return trainer.transformer_config(5, batch=4, seq_len=8, vocab=50, embed_dim=16, heads=2, blocks=2,
                                      ffn=32, classes=4)


def test_cnet_layout_mlp(gpu, tmp_path):
    cfg = _mlp_cfg()
    print("[ckpt] cnet layout mlp", flush=True)
    params, X, Y = trainer.synthetic_mlp(cfg, np.random.default_rng(1))
    s = trainer.Session(cfg)
    s.set_params(params)
    s.set_batch(X, Y)
    s.step()
    s.save_model(tmp_path / "m.cnet")
    buf = (tmp_path / "m.cnet").read_bytes()
    nlayers, recs, end = _parse_cnet(buf)
    assert end == len(buf)
    assert [t for t, _ in recs] == [1, 1, 1]
    got = s.get_params()
    for i, (_, tensors) in enumerate(recs):
        (wd, w), (bd, b) = tensors
        assert wd == [cfg.sizes[i], cfg.sizes[i + 1]] and bd == [cfg.sizes[i + 1]]
        np.testing.assert_array_equal(w, got[2 * i])
        np.testing.assert_array_equal(b, got[2 * i + 1])
    s.close()


def test_load_handbuilt_cnet(gpu, tmp_path):
    """A file written from the reference's format description, not by our writer."""
    cfg = _mlp_cfg()
    print("[ckpt] hand-built cnet", flush=True)
    rng = np.random.default_rng(2)
    params = [rng.standard_normal(p.size).astype(np.float32)
              for p in trainer.synthetic_mlp(cfg, rng)[0]]
    body = b""
    for i in range(3):
        body += struct.pack("<i", 1) + _put([cfg.sizes[i], cfg.sizes[i + 1]], params[2 * i])
        body += _put([cfg.sizes[i + 1]], params[2 * i + 1])
    # layer count as the reference writes it (all layers, activations included)
    (tmp_path / "h.cnet").write_bytes(struct.pack("<ii", MAGIC, 5) + body)
    s = trainer.Session(cfg)
    s.load_model(tmp_path / "h.cnet")
    for a, b in zip(s.get_params(), params):
        np.testing.assert_array_equal(a, b)
    (tmp_path / "bad.cnet").write_bytes(struct.pack("<ii", 0x1234, 1))
    with pytest.raises(Exception, match="bad magic"):
        s.load_model(tmp_path / "bad.cnet")
    s.close()


def test_cnet_layout_transformer(gpu, tmp_path):
    """Embedding (type 3, [vocab, dim]), per block MHA (type 0: no data, as the
    reference), BatchNorm (type 2: gamma, beta, running mean and var), two
    Linear (type 1), then the classifier; loading restores exactly those."""
    cfg = _tf_cfg()
    print("[ckpt] cnet layout transformer", flush=True)
    params, ids, Y = trainer.synthetic_transformer(cfg, np.random.default_rng(3))
    s = trainer.Session(cfg)
    s.set_params(params)
    s.set_batch(ids, Y)
    s.step()
    s.save_model(tmp_path / "t.cnet")
    buf = (tmp_path / "t.cnet").read_bytes()
    _, recs, end = _parse_cnet(buf)
    assert end == len(buf)
    assert [t for t, _ in recs] == [3] + [0, 2, 1, 1] * cfg.blocks + [1]
    got = s.get_params()
    assert recs[0][1][0][0] == [cfg.vocab, cfg.embed_dim]
    np.testing.assert_array_equal(recs[0][1][0][1], got[0])
    per_block = 10  # W_q, W_k, W_v, W_o, gamma, beta, W1, b1, W2, b2
    for blk in range(cfg.blocks):
        base = 1 + blk * per_block
        bn = recs[1 + 4 * blk + 1][1]
        np.testing.assert_array_equal(bn[0][1], got[base + 4])
        np.testing.assert_array_equal(bn[1][1], got[base + 5])
        assert bn[3][1].min() > 0  # running variance after one training step
        for j, li in enumerate((2, 3)):
            w, b = recs[1 + 4 * blk + li][1]
            np.testing.assert_array_equal(w[1], got[base + 6 + 2 * j])
            np.testing.assert_array_equal(b[1], got[base + 7 + 2 * j])
    fresh = trainer.Session(_tf_cfg_seed(cfg, 99))
    fresh.load_model(tmp_path / "t.cnet")
    after = fresh.get_params()
    for k in range(len(got)):
        in_block = (k - 1) % per_block if 1 <= k < 1 + cfg.blocks * per_block else None
        if in_block is not None and in_block < 4:
            continue  # MHA weights: type 0 records carry none
        np.testing.assert_array_equal(after[k], got[k])
    s.close()
    fresh.close()


def _tf_cfg_seed(cfg, seed):
    c = _tf_cfg()
    c.seed = seed
    return c


RESUME = {
    "mlp_adam": lambda: (_mlp_cfg(), trainer.synthetic_mlp),
    "mlp_rmsprop": lambda: (_mlp_cfg("rmsprop"), trainer.synthetic_mlp),
    "cnn_momentum": lambda: (_opt(trainer.cnn_config(3, batch=8), "momentum"), trainer.synthetic_cnn),
    "lstm_adam": lambda: (trainer.rnn_config(4, batch=8, seq_len=6), trainer.synthetic_rnn),
    "elman_adagrad": lambda: (_opt(trainer.rnn_config(4, batch=8, seq_len=6, cell="rnn"), "adagrad"),
                              trainer.synthetic_rnn),
    "transformer_adam": lambda: (_tf_cfg(), trainer.synthetic_transformer),
    # the Dropout layers' mask positions travel with the checkpoint
    "mlp_dropout_adam": lambda: (_dropout_cfg(), trainer.synthetic_mlp),
}


def _dropout_cfg():
    cfg = _mlp_cfg()
    cfg.dropout = 0.3
    return cfg


def _opt(cfg, opt):
    cfg.optimizer, cfg.opt_hyper, cfg.opt_eps = opt, 0.9, 1e-8
    return cfg


def _bits(a):
    return np.atleast_1d(np.asarray(a, np.float32)).view(np.uint32)


@pytest.mark.parametrize("name", list(RESUME))
def test_checkpoint_resumes_exactly(gpu, tmp_path, name):
    cfg, synth = RESUME[name]()
    print(f"[ckpt] resume {name}", flush=True)
    rng = np.random.default_rng(21)
    params, X0, Y0 = synth(cfg, rng)
    batches = [synth(cfg, rng)[1:] for _ in range(6)]
    a = trainer.Session(cfg)
    a.set_params(params)
    for X, Y in batches[:3]:
        a.set_batch(X, Y)
        a.step()
    path = tmp_path / f"{name}.ckpt"
    a.save_checkpoint(path)
    a.save_model(tmp_path / f"{name}.cnet")
    # the checkpoint begins with the reference's model file
    cnet = (tmp_path / f"{name}.cnet").read_bytes()
    assert path.read_bytes()[:len(cnet)] == cnet
    cfg.seed += 1000  # other initial weights
    b = trainer.Session(cfg)
    b.load_checkpoint(path)
    for pa, pb in zip(a.get_params(), b.get_params()):
        np.testing.assert_array_equal(_bits(pa), _bits(pb))
    for k, (X, Y) in enumerate(batches[3:]):
        a.set_batch(X, Y)
        b.set_batch(X, Y)
        la, lb = a.step(), b.step()
        assert _bits(la)[0] == _bits(lb)[0], f"step {k + 3}: loss {lb!r} (loaded) vs {la!r}"
    for i, (pa, pb) in enumerate(zip(a.get_params(), b.get_params())):
        assert np.array_equal(_bits(pa), _bits(pb)), f"parameter {i} differs after resuming"
    a.close()
    b.close()


def _refused_load_changes_nothing(cfg, path, match, X, Y):
    """A refused load leaves the session's parameters and its training run as
    they were: the next step equals that of an untouched twin session."""
    params = trainer.synthetic_mlp(cfg, np.random.default_rng(99))[0]
    s, twin = trainer.Session(cfg), trainer.Session(cfg)
    for x in (s, twin):
        x.set_params(params)
        x.set_batch(X, Y)
        x.step()
    with pytest.raises(Exception, match=match):
        s.load_checkpoint(path)
    for k, (a, b) in enumerate(zip(s.get_params(), twin.get_params())):
        assert np.array_equal(_bits(a), _bits(b)), f"parameter {k} changed by a refused load"
    assert _bits(s.step())[0] == _bits(twin.step())[0]  # optimizer state untouched too
    for k, (a, b) in enumerate(zip(s.get_params(), twin.get_params())):
        assert np.array_equal(_bits(a), _bits(b)), f"parameter {k} differs one step after a refused load"
    s.close()
    twin.close()


def test_checkpoint_refuses_other_optimizer_and_shapes(gpu, tmp_path):
    cfg = _mlp_cfg()
    print("[ckpt] refusals", flush=True)
    params, X, Y = trainer.synthetic_mlp(cfg, np.random.default_rng(4))
    a = trainer.Session(cfg)
    a.set_batch(X, Y)
    a.step()
    a.save_checkpoint(tmp_path / "a.ckpt")
    # an Adam checkpoint into an SGD session: every CNET record fits, the
    # optimizer section does not -- nothing may be written
    sgd = _mlp_cfg("sgd")
    _refused_load_changes_nothing(sgd, tmp_path / "a.ckpt", "kind", X, Y)
    # the first two Linear records fit, the third does not
    other = trainer.MLPConfig("MLP 20-32-16-4", [20, 32, 16, 4], "relu", "none", "softmax_ce", 24)
    _, Xo, Yo = trainer.synthetic_mlp(other, np.random.default_rng(5))
    _refused_load_changes_nothing(other, tmp_path / "a.ckpt", "hape", Xo, Yo)
    # a plain model file has no extension
    _refused_load_changes_nothing(cfg, _save_plain(a, tmp_path), "extension", X, Y)
    # a checkpoint with Dropout generators into a model without Dropout layers
    d = trainer.Session(_dropout_cfg())
    d.set_batch(X, Y)
    d.step()
    d.save_checkpoint(tmp_path / "d.ckpt")
    _refused_load_changes_nothing(cfg, tmp_path / "d.ckpt", "Dropout", X, Y)
    # a file cut 1-3 bytes into the Dropout section's tag is a truncated file,
    # not an older checkpoint without that section
    raw = (tmp_path / "d.ckpt").read_bytes()
    tag = raw.rfind(struct.pack("<i", 0x434E5253))
    assert tag > 0
    for cut in (1, 2, 3):
        (tmp_path / f"cut{cut}.ckpt").write_bytes(raw[:tag + cut])
        _refused_load_changes_nothing(_dropout_cfg(), tmp_path / f"cut{cut}.ckpt", "Truncated", X, Y)
    # cut exactly before the tag: a checkpoint written before the section
    # existed, which loads and leaves the generators as they are
    (tmp_path / "cut0.ckpt").write_bytes(raw[:tag])
    e = trainer.Session(_dropout_cfg())
    e.load_checkpoint(tmp_path / "cut0.ckpt")
    e.close()
    d.close()
    a.close()


def test_dropout_model_refuses_capture(gpu):
    cfg = _dropout_cfg()
    params, X, Y = trainer.synthetic_mlp(cfg, np.random.default_rng(6))
    s = trainer.Session(cfg)
    s.set_batch(X, Y)
    s.step()
    with pytest.raises(Exception, match="Dropout"):
        s.capture()
    s.close()


def _save_plain(sess, tmp_path):
    p = tmp_path / "plain.cnet"
    sess.save_model(p)
    return p
