"""GPU parity of LSTM / GRU forward and BPTT against the CPU oracle.

Outputs, caches and gradients within rel 1e-4 / abs 1e-5.  The weight and
input gradients are contractions over B*S rows (the reference sums the same
terms per timestep), so their relative part is taken against the RMS size
of the partial sums (oracle_lib.close_mag, magnitudes from |operands|).
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


def _inputs(rng, B, S, I, H, G):
    X = rng.standard_normal(B * S * I).astype(np.float32)
    lih, lhh = np.sqrt(6.0 / (I + H)), np.sqrt(6.0 / (2 * H))  # lstm.cpp:42-45 limits
    Wih = rng.uniform(-lih, lih, I * G * H).astype(np.float32)
    Whh = rng.uniform(-lhh, lhh, H * G * H).astype(np.float32)
    b = (rng.standard_normal(G * H) * 0.1).astype(np.float32)
    dY = (rng.standard_normal(B * S * H) * 1e-2).astype(np.float32)
    return X, Wih, Whh, b, dY


RNN_CASES = [(3, 5, 4, 8), (8, 7, 16, 32), (5, 1, 3, 6), (40, 6, 12, 71), (128, 64, 128, 512)]
# shapes the persistent recurrence takes (B % 16 == 0, H one of 64, 128, 256,
# 512, S >= 2): one XCD's sample tile, three of eight XCDs, all eight, two
# sample tiles per XCD
PERSIST_CASES = [(16, 5, 8, 64), (48, 9, 24, 128), (128, 64, 128, 512), (256, 6, 32, 256)]
# shapes whose persistent backward also accumulates the weight gradients
# (I = 64 or 128): each hidden size, W_hh in registers (H <= 256) and in LDS
# (H = 512), one and two 64-wide input tiles, one and several sample tiles
FUSED_CASES = [(32, 7, 64, 64), (48, 4, 128, 128), (64, 5, 128, 256), (16, 3, 64, 512), (128, 64, 128, 512)]
LSTM_CASES = ([(*c, "per-step") for c in RNN_CASES if c not in PERSIST_CASES] +
              [(*c, path) for c in PERSIST_CASES for path in ("persistent", "per-step")] +
              [(*c, path) for c in FUSED_CASES for path in ("persistent", "persistent-unfused")
               if (*c, path) not in [(*p, "persistent") for p in PERSIST_CASES]])


@pytest.mark.parametrize("B,S,I,H,path", LSTM_CASES)
def test_lstm_vs_oracle(gpu, oracle, monkeypatch, B, S, I, H, path):
    """Both recurrence paths -- one persistent launch for all timesteps, or
    one launch per timestep -- against the oracle (they sum the recurrent
    products in different orders, so each is held to the oracle's bars).
    Where I is 64 or 128 the persistent forward computes the input
    projection and the persistent backward the weight gradients itself
    ("persistent"), or leaves them to the GEMMs ("persistent-unfused")."""
    print(f"[lstm] B={B} S={S} I={I} H={H} {path}", flush=True)
    monkeypatch.setenv("CNHIP_RECURRENCE_PERSISTENT", "0" if path == "per-step" else "1")
    monkeypatch.setenv("CNHIP_RECURRENCE_FUSED_DW", "0" if path == "persistent-unfused" else "1")
    monkeypatch.setenv("CNHIP_RECURRENCE_FUSED_X", "0" if path == "persistent-unfused" else "1")
    oracle.cnref_set_threads(16)
    rng = np.random.default_rng(B + S + I + H)
    X, Wih, Whh, b, dY = _inputs(rng, B, S, I, H, 4)
    b[H:2 * H] += 1.0  # forget bias (lstm.cpp:47-49)
    BS, G = B * S, 4 * H
    Y, gates = torch.empty(BS * H, device="cuda"), torch.empty(BS * G, device="cuda")
    c, tc = torch.empty(BS * H, device="cuda"), torch.empty(BS * H, device="cuda")
    # a 3-block launch first: the next grid's blocks are then dealt to the
    # XCDs from another starting XCD (the persistent kernels place their
    # tiles by the XCD each block runs on, not by block index)
    odd = torch.ones(3 * 256, device="cuda")
    ops.relu_forward(odd, torch.empty_like(odd))
    ops.lstm_forward(dev(X), dev(Wih), dev(Whh), dev(b), Y, gates, c, tc, B, S, I, H)
    gWih, gWhh = torch.empty(I * G, device="cuda"), torch.empty(H * G, device="cuda")
    gb, dX = torch.empty(G, device="cuda"), torch.empty(BS * I, device="cuda")
    ops.relu_forward(odd, torch.empty_like(odd))
    ops.lstm_backward(dev(X), dev(Wih), dev(Whh), Y, gates, c, tc, dev(dY), gWih, gWhh, gb, dX,
                      B, S, I, H)
    rY, rg = np.zeros(BS * H, np.float32), np.zeros(BS * G, np.float32)
    rc, rtc = np.zeros(BS * H, np.float32), np.zeros(BS * H, np.float32)
    oracle.cnref_lstm_forward(fp(X), fp(Wih), fp(Whh), fp(b), fp(rY), fp(rg), fp(rc), fp(rtc), B, S, I, H)
    for got, want, name in [(host(Y), rY, "Y"), (host(gates), rg, "gates"), (host(c), rc, "c")]:
        ok, msg = close(got, want, 1e-4, 2e-5)
        assert ok, f"{name}: {msg}"
    # backward on the oracle's own caches, so forward rounding does not leak in
    rgWih, rgWhh = np.zeros(I * G, np.float32), np.zeros(H * G, np.float32)
    rgb, rdX = np.zeros(G, np.float32), np.zeros(BS * I, np.float32)
    oracle.cnref_lstm_backward(fp(X), fp(Wih), fp(Whh), fp(rY), fp(rg), fp(rc), fp(rtc), fp(dY),
                               fp(rgWih), fp(rgWhh), fp(rgb), fp(rdX), B, S, I, H)
    # magnitudes of the final contractions: dG is bounded by |dY| * O(S) here
    dGabs = np.full(BS * G, np.abs(dY).mean() * 4, np.float32)
    m_ih = gemm_mag(oracle, 1, 0, I, G, BS, X, BS, dGabs, BS, I)
    m_hh = gemm_mag(oracle, 1, 0, H, G, BS, np.abs(rY), BS, dGabs, BS, H)
    m_b = gemm_mag(oracle, 1, 0, 1, G, BS, np.ones(BS, np.float32), BS, dGabs, BS, 1)
    m_dx = gemm_mag(oracle, 0, 1, BS, I, G, dGabs, BS, Wih, I, BS)
    for got, want, mag, name in [(host(gWih), rgWih, m_ih, "grad_W_ih"),
                                 (host(gWhh), rgWhh, m_hh, "grad_W_hh"),
                                 (host(gb), rgb, m_b, "grad_b"), (host(dX), rdX, m_dx, "dX")]:
        ok, msg = close_mag(got, want, mag, 1e-4, 1e-5)
        assert ok, f"{name}: {msg}"


@pytest.mark.parametrize("B,S,I,H", RNN_CASES[:3] + [(64, 32, 64, 256)])
def test_gru_vs_oracle(gpu, oracle, B, S, I, H):
    print(f"[gru] B={B} S={S} I={I} H={H}", flush=True)
    oracle.cnref_set_threads(16)
    rng = np.random.default_rng(B * 3 + S + I + H)
    X, Wih, Whh, b, dY = _inputs(rng, B, S, I, H, 3)
    BS, G = B * S, 3 * H
    Y, gates, rh = (torch.empty(BS * H, device="cuda"), torch.empty(BS * G, device="cuda"),
                    torch.empty(BS * H, device="cuda"))
    ops.gru_forward(dev(X), dev(Wih), dev(Whh), dev(b), Y, gates, rh, B, S, I, H)
    gWih, gWhh = torch.empty(I * G, device="cuda"), torch.empty(H * G, device="cuda")
    gb, dX = torch.empty(G, device="cuda"), torch.empty(BS * I, device="cuda")
    ops.gru_backward(dev(X), dev(Wih), dev(Whh), Y, gates, rh, dev(dY), gWih, gWhh, gb, dX, B, S, I, H)
    rY, rg, rrh = np.zeros(BS * H, np.float32), np.zeros(BS * G, np.float32), np.zeros(BS * H, np.float32)
    oracle.cnref_gru_forward(fp(X), fp(Wih), fp(Whh), fp(b), fp(rY), fp(rg), fp(rrh), B, S, I, H)
    for got, want, name in [(host(Y), rY, "Y"), (host(gates), rg, "gates"), (host(rh), rrh, "rh")]:
        ok, msg = close(got, want, 1e-4, 2e-5)
        assert ok, f"{name}: {msg}"
    rgWih, rgWhh = np.zeros(I * G, np.float32), np.zeros(H * G, np.float32)
    rgb, rdX = np.zeros(G, np.float32), np.zeros(BS * I, np.float32)
    oracle.cnref_gru_backward(fp(X), fp(Wih), fp(Whh), fp(rY), fp(rg), fp(rrh), fp(dY), fp(rgWih),
                              fp(rgWhh), fp(rgb), fp(rdX), B, S, I, H)
    dGabs = np.full(BS * G, np.abs(dY).mean() * 4, np.float32)
    m_ih = gemm_mag(oracle, 1, 0, I, G, BS, X, BS, dGabs, BS, I)
    m_hh = gemm_mag(oracle, 1, 0, H, G, BS, np.abs(rY) + 1e-3, BS, dGabs, BS, H)
    m_b = gemm_mag(oracle, 1, 0, 1, G, BS, np.ones(BS, np.float32), BS, dGabs, BS, 1)
    m_dx = gemm_mag(oracle, 0, 1, BS, I, G, dGabs, BS, Wih, I, BS)
    for got, want, mag, name in [(host(gWih), rgWih, m_ih, "grad_W_ih"),
                                 (host(gWhh), rgWhh, m_hh, "grad_W_hh"),
                                 (host(gb), rgb, m_b, "grad_b"), (host(dX), rdX, m_dx, "dX")]:
        ok, msg = close_mag(got, want, mag, 1e-4, 1e-5)
        assert ok, f"{name}: {msg}"


def test_seq_select_scatter(gpu):
    B, S, D = 5, 4, 3
    Y = torch.arange(B * S * D, dtype=torch.float32, device="cuda")
    out = torch.empty(B * D, device="cuda")
    ops.seq_select(Y, out, B, S, D, S - 1)
    y = Y.cpu().numpy().reshape(D, S, B).transpose(2, 1, 0)
    np.testing.assert_array_equal(host(out).reshape(D, B).T, y[:, S - 1, :])
    back = torch.full((B * S * D,), 7.0, device="cuda")
    ops.seq_scatter(out, back, B, S, D, S - 1)
    b = host(back).reshape(D, S, B).transpose(2, 1, 0)
    assert not b[:, :S - 1, :].any()
    np.testing.assert_array_equal(b[:, S - 1, :], y[:, S - 1, :])


def _lstm_run(B, S, I, H, seed, env, backward=True):
    """forward (+ backward) with the given CNHIP_* environment; host copies."""
    import os
    saved = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        rng = np.random.default_rng(seed)
        X, Wih, Whh, b, dY = _inputs(rng, B, S, I, H, 4)
        BS, G = B * S, 4 * H
        Y, gates = torch.empty(BS * H, device="cuda"), torch.empty(BS * G, device="cuda")
        c, tc = torch.empty(BS * H, device="cuda"), torch.empty(BS * H, device="cuda")
        ops.lstm_forward(dev(X), dev(Wih), dev(Whh), dev(b), Y, gates, c, tc, B, S, I, H)
        if not backward:
            return [host(t) for t in (Y, gates, c, tc)]
        gWih, gWhh = torch.empty(I * G, device="cuda"), torch.empty(H * G, device="cuda")
        gb, dX = torch.empty(G, device="cuda"), torch.empty(BS * I, device="cuda")
        ops.lstm_backward(dev(X), dev(Wih), dev(Whh), Y, gates, c, tc, dev(dY), gWih, gWhh, gb, dX, B, S, I, H)
        return [host(t) for t in (Y, gates, c, tc, gWih, gWhh, gb, dX)]
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def test_lstm_persistent_wait_fault_is_reported(gpu):
    """Forced from the host: with a negative spin limit every wait of the
    persistent recurrence gives up at once, so every block exits normally;
    the launch's fault is reported by the next recurrent call, once, and the
    run after it is correct again."""
    from cppnet_amd import _capi
    B, S, I, H = 64, 6, 16, 128
    print("[lstm-persist] forced wait fault", flush=True)
    # the faulted forward launch's own call returns before the GPU has run it
    _lstm_run(B, S, I, H, 3, {"CNHIP_RECURRENCE_SPIN_LIMIT": "-1", "CNHIP_RECURRENCE_PERSISTENT": "1"},
              backward=False)
    torch.cuda.synchronize()
    with pytest.raises(_capi.CnhipError, match="gave up waiting"):
        _lstm_run(B, S, I, H, 3, {"CNHIP_RECURRENCE_PERSISTENT": "1"})
    torch.cuda.synchronize()
    good = _lstm_run(B, S, I, H, 3, {"CNHIP_RECURRENCE_PERSISTENT": "1"})
    again = _lstm_run(B, S, I, H, 3, {"CNHIP_RECURRENCE_PERSISTENT": "1"})
    ref = _lstm_run(B, S, I, H, 3, {"CNHIP_RECURRENCE_PERSISTENT": "0"})
    for x, y in zip(good, again):  # deterministic: fixed summation order
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
    for x, y, name in zip(good[:4], ref[:4], ["Y", "gates", "c", "tanh_c"]):
        ok, msg = close(x, y, 1e-4, 2e-5)
        assert ok, f"{name}: persistent vs per-step: {msg}"


def test_lstm_persistent_exchange_reuse_is_exact(gpu):
    """Launch after launch the persistent kernels reuse their exchange area
    without zeroing it (each launch stamps its words with a new epoch): runs
    of one shape repeat bit for bit, also after a larger shape has grown the
    area and a different layout (forward vs backward) has written over it."""
    env = {"CNHIP_RECURRENCE_PERSISTENT": "1"}
    print("[lstm-persist] exchange reuse", flush=True)
    first = _lstm_run(64, 6, 64, 128, 5, env)
    for shape in [(64, 6, 64, 128), (128, 9, 128, 256), (64, 6, 64, 128), (32, 4, 16, 64), (64, 6, 64, 128)]:
        got = _lstm_run(*shape, 5, env)
        if shape == (64, 6, 64, 128):
            for x, y in zip(first, got):
                assert np.array_equal(x.view(np.uint32), y.view(np.uint32))


def test_lstm_persistent_config4_shape_repeats_bit_for_bit(gpu):
    """At config 4's shape (8 sample tiles of 32 blocks each, W_hh in LDS,
    the weight gradients accumulated in the backward) three runs of the
    persistent forward and backward give the same bits: every exchanged
    value is taken with its own step's stamp, and every sum has a fixed
    order."""
    env = {"CNHIP_RECURRENCE_PERSISTENT": "1", "CNHIP_RECURRENCE_FUSED_DW": "1", "CNHIP_RECURRENCE_FUSED_X": "1"}
    print("[lstm-persist] config 4 shape, 3 runs", flush=True)
    runs = [_lstm_run(128, 64, 128, 512, 11, env) for _ in range(3)]
    names = ["Y", "gates", "c", "tanh_c", "grad_W_ih", "grad_W_hh", "grad_b", "dX"]
    for other in runs[1:]:
        for x, y, name in zip(runs[0], other, names):
            assert np.array_equal(x.view(np.uint32), y.view(np.uint32)), f"{name} differs between runs"


@pytest.mark.parametrize("B,S,I,H,path", [(32, 7, 64, 64, "persistent"), (128, 64, 128, 512, "persistent"),
                                          (48, 9, 24, 128, "persistent"), (32, 7, 64, 64, "persistent-unfused"),
                                          (40, 6, 12, 71, "per-step")])
def test_lstm_backward_last_step_gradient(gpu, monkeypatch, B, S, I, H, path):
    """cnhip_lstm_backward_last (the gradient of the last step's output only,
    as an LSTM -> SequenceLast model passes it) against the same gradient
    spread over all steps with zeros and cnhip_lstm_backward: bit for bit."""
    print(f"[lstm-last] B={B} S={S} I={I} H={H} {path}", flush=True)
    monkeypatch.setenv("CNHIP_RECURRENCE_PERSISTENT", "0" if path == "per-step" else "1")
    monkeypatch.setenv("CNHIP_RECURRENCE_FUSED_DW", "0" if path == "persistent-unfused" else "1")
    monkeypatch.setenv("CNHIP_RECURRENCE_FUSED_X", "0" if path == "persistent-unfused" else "1")
    rng = np.random.default_rng(B * S + H)
    X, Wih, Whh, b, _ = _inputs(rng, B, S, I, H, 4)
    BS, G = B * S, 4 * H
    Y, gates = torch.empty(BS * H, device="cuda"), torch.empty(BS * G, device="cuda")
    c, tc = torch.empty(BS * H, device="cuda"), torch.empty(BS * H, device="cuda")
    ops.lstm_forward(dev(X), dev(Wih), dev(Whh), dev(b), Y, gates, c, tc, B, S, I, H)
    dlast = (rng.standard_normal(B * H) * 1e-2).astype(np.float32)
    full = np.zeros((H, S, B), np.float32)  # ColMajor [B, S, H]
    full[:, S - 1, :] = dlast.reshape(H, B)
    outs = []
    for fn, dy in [(ops.lstm_backward, full.reshape(-1)), (ops.lstm_backward_last, dlast)]:
        gWih, gWhh = torch.empty(I * G, device="cuda"), torch.empty(H * G, device="cuda")
        gb, dX = torch.empty(G, device="cuda"), torch.empty(BS * I, device="cuda")
        fn(dev(X), dev(Wih), dev(Whh), Y, gates, c, tc, dev(dy), gWih, gWhh, gb, dX, B, S, I, H)
        outs.append([host(t) for t in (gWih, gWhh, gb, dX)])
    for x, y, name in zip(outs[0], outs[1], ["grad_W_ih", "grad_W_hh", "grad_b", "dX"]):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32)), name


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _snapshot(sess):
    m, t = sess.get_opt_state(0)
    v, _ = sess.get_opt_state(1)
    return sess.get_params(), m, v, t


def _assert_same(a, b, what):
    pa, ma, va, ta = a
    pb, mb, vb, tb = b
    assert ta == tb, f"{what}: Adam step counts {tb} vs {ta}"
    for k in range(len(pa)):
        for u, w, name in ((pa[k], pb[k], "value"), (ma[k], mb[k], "m"), (va[k], vb[k], "v")):
            assert np.array_equal(_bits(u), _bits(w)), f"{what}: {name} of parameter {k} differs"


@pytest.mark.parametrize("read_loss", [True, False])
def test_lstm_fault_in_training_step_withholds_the_update(gpu, monkeypatch, read_loss):
    """A persistent recurrence launch that gives up (forced from the host:
    spin limit -1, so every block exits at once) inside a full config-4
    training step (LSTM 128->512, T 64, B 128 -> Linear -> MSE -> Adam),
    with no synchronization between the backward and the update: the device
    withholds the step's Adam launch, the step reports the fault (at its
    loss read-back; without one, at the next step or sync), the parameters,
    m, v and Adam's per-key t are exactly as before the step, and training
    continues bit for bit as a session that never faulted."""
    from cppnet_amd import _capi, trainer
    print(f"[lstm-fault] config-4 step, read_loss={read_loss}", flush=True)
    monkeypatch.setenv("CNHIP_RECURRENCE_PERSISTENT", "1")
    cfg = trainer.rnn_config(4)
    rng = np.random.default_rng(44)
    params, X, Y = trainer.synthetic_rnn(cfg, rng)
    a, twin = trainer.Session(cfg), trainer.Session(cfg)
    for s in (a, twin):
        s.set_params(params)
        s.set_batch(X, Y)
        s.step()
        s.step()
    before = _snapshot(a)
    _assert_same(before, _snapshot(twin), "twin sessions")
    monkeypatch.setenv("CNHIP_RECURRENCE_SPIN_LIMIT", "-1")
    raised = False
    try:
        if read_loss:
            a.step()  # the fault surfaces at this step's own loss read-back
        else:
            a.step(read_loss=False)
            monkeypatch.delenv("CNHIP_RECURRENCE_SPIN_LIMIT")
            a.step(read_loss=False)  # either this step or the sync reports it
            a.synchronize()
    except _capi.CnhipError as e:
        assert "gave up waiting" in str(e), str(e)
        raised = True
    monkeypatch.delenv("CNHIP_RECURRENCE_SPIN_LIMIT", raising=False)
    assert raised, "the faulted step was not reported"
    a.synchronize()  # nothing left pending
    _assert_same(before, _snapshot(a), "after the faulted step")
    la, lt = a.step(), twin.step()
    assert _bits(la)[0] == _bits(lt)[0], f"loss after the fault {la!r} vs {lt!r}"
    _assert_same(_snapshot(twin), _snapshot(a), "one step after the fault")
    a.close()
    twin.close()
