"""GPU parity of the transformer-row ops (MultiHeadAttention, Embedding,
BatchNorm, GELU, MeanPool1D, residual add, transpose) against the CPU oracle.

Bars: embedding routing, its deterministic scatter-add (same addition order
as the reference's cpu-eigen loop), transpose and the mean-pool broadcast are
bit-exact; everything else within rel 1e-4 / abs 1e-5, where the relative
part of a contraction is taken against the RMS size of its partial sums
(oracle_lib.close_mag; for attention the magnitudes are chained through the
intermediate products in float64).
"""
import numpy as np
import pytest
import torch

from cppnet_amd import ops
from oracle_lib import close, close_mag, fp
from oracle import ip

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def cm(a):
    a = np.asarray(a)
    return np.ascontiguousarray(a.transpose(*reversed(range(a.ndim)))).ravel()


def from_cm(flat, shape):
    return np.asarray(flat).reshape(tuple(reversed(shape))).transpose(*reversed(range(len(shape))))


@pytest.mark.parametrize("R,C", [(1, 1), (63, 65), (64, 64), (130, 7), (4096, 33), (32, 131072), (16, 1024),
                                 (128, 32), (8192, 512), (36, 100), (20, 12), (12, 20)])
def test_transpose_exact(gpu, R, C):
    print(f"[transpose] {R}x{C}", flush=True)
    a = np.random.default_rng(R * C).standard_normal(R * C).astype(np.float32)
    out = torch.empty(R * C, device="cuda")
    ops.transpose(dev(a), out, R, C)
    np.testing.assert_array_equal(host(out), cm(from_cm(a, (R, C)).T))


# ---------------------------------------------------------------- attention
def _mha_logical(x3, Ws, dy, heads):
    """float64 intermediates and per-output magnitudes (RMS partial sums,
    chained through the products) of single-head full-width attention."""
    q, k, v = x3
    Wq, Wk, Wv, Wo = Ws
    D, S = Wq.shape[0], q.shape[1]
    sc = 1.0 / np.sqrt(np.float32(D // heads))
    Qp, Kp, Vp = q @ Wq, k @ Wk, v @ Wv
    z = Qp @ Kp.transpose(0, 2, 1) * sc
    A = np.exp(z - z.max(-1, keepdims=True))
    A /= A.sum(-1, keepdims=True)
    ctx = A @ Vp
    aq, ak, av = np.abs(q), np.abs(k), np.abs(v)
    aWq, aWk, aWv, aWo = (np.abs(w) for w in Ws)
    mQ, mK, mV = aq @ aWq / np.sqrt(D), ak @ aWk / np.sqrt(D), av @ aWv / np.sqrt(D)
    mz = (mQ @ mK.transpose(0, 2, 1) / np.sqrt(D)) * sc
    mctx = A @ mV + (A * mz) @ np.abs(Vp) / np.sqrt(S)
    m = {"out": (mctx @ aWo) / np.sqrt(D)}
    gctx = dy @ Wo.T
    mg = np.abs(dy) @ aWo.T / np.sqrt(D)
    gA = gctx @ Vp.transpose(0, 2, 1)
    mgA = (mg @ np.abs(Vp).transpose(0, 2, 1) + np.abs(gctx) @ mV.transpose(0, 2, 1)) / np.sqrt(D)
    mgS = (A * (mgA + (mgA * A).sum(-1, keepdims=True)) + A * mz * np.abs(gA)) * sc
    mgQ = (mgS @ np.abs(Kp) + np.abs(mgS) @ mK) / np.sqrt(S)
    mgK = (mgS.transpose(0, 2, 1) @ np.abs(Qp) + mgS.transpose(0, 2, 1) @ mQ) / np.sqrt(S)
    mgV = (A.transpose(0, 2, 1) @ mg) / np.sqrt(S)
    BS = q.shape[0] * S
    flat = lambda t: t.reshape(BS, -1)  # noqa: E731
    m["gWo"] = flat(np.abs(ctx) + mctx).T @ flat(np.abs(dy)) / np.sqrt(BS)
    m["gWq"] = flat(aq).T @ flat(mgQ) / np.sqrt(BS)
    m["gWk"] = flat(ak).T @ flat(mgK) / np.sqrt(BS)
    m["gWv"] = flat(av).T @ flat(mgV) / np.sqrt(BS)
    m["dX"] = (mgQ @ aWq.T + mgK @ aWk.T + mgV @ aWv.T) / np.sqrt(3 * D)
    return m


MHA_CASES = [(2, 5, 8, 2), (3, 7, 12, 4), (4, 33, 64, 8), (8, 256, 512, 8)]


@pytest.mark.parametrize("self_attn", [True, False])
@pytest.mark.parametrize("B,S,D,h", MHA_CASES)
def test_mha_vs_oracle(gpu, oracle, B, S, D, h, self_attn):
    print(f"[mha] B={B} S={S} D={D} heads={h} self={self_attn}", flush=True)
    oracle.cnref_set_threads(16)
    rng = np.random.default_rng(B * 7 + S + D + self_attn)
    lim = np.sqrt(6.0 / (2 * D))  # attention.cpp:47-50 xavier limit
    Ws = [rng.uniform(-lim, lim, (D, D)).astype(np.float32) for _ in range(4)]
    xs = [rng.standard_normal((B, S, D)).astype(np.float32) for _ in range(1 if self_attn else 3)]
    if self_attn:
        xs = xs * 3
    dy = (rng.standard_normal((B, S, D)) * 1e-2).astype(np.float32)
    X = [cm(x) for x in xs]
    Wc = [cm(w) for w in Ws]
    # device: packed weights [Wq | Wk | Wv | Wo] (adjacent D*D blocks) for the
    # self-attention case, separate tensors otherwise
    if self_attn:
        Wall = dev(np.concatenate(Wc))
        Wd = [Wall[i * D * D:(i + 1) * D * D] for i in range(4)]
        gall = torch.full((4 * D * D,), 7.0, device="cuda")
        gW = [gall[i * D * D:(i + 1) * D * D] for i in range(4)]
        xd = [dev(X[0])] * 3
    else:
        Wd = [dev(w) for w in Wc]
        gW = [torch.full((D * D,), 7.0, device="cuda") for _ in range(4)]
        xd = [dev(x) for x in X]
    out = torch.empty(B * S * D, device="cuda")
    cache = torch.empty(ops.mha_cache_floats(B, S, D), device="cuda")
    ops.mha_forward(*xd, *Wd, out, cache, B, S, D, h)
    dX = torch.empty(B * S * D, device="cuda")
    ops.mha_backward(*xd, *Wd, cache, dev(cm(dy)), *gW, dX, B, S, D, h)
    r_out, r_attn = np.zeros(B * S * D, np.float32), np.zeros(B * S * S, np.float32)
    oracle.cnref_mha_forward(*[fp(x) for x in X], *[fp(w) for w in Wc],
                             fp(r_out), fp(r_attn), B, S, D, h)
    r_g = [np.zeros(D * D, np.float32) for _ in range(4)]
    r_dX = np.zeros(B * S * D, np.float32)
    oracle.cnref_mha_backward(*[fp(x) for x in X], *[fp(w) for w in Wc],
                              fp(r_attn), fp(cm(dy)), *[fp(a) for a in r_g], fp(r_dX), B, S, D, h)
    x64 = [x.astype(np.float64) for x in xs]
    mags = _mha_logical(x64, [w.astype(np.float64) for w in Ws], dy.astype(np.float64), h)
    # attention weights from the cache: sample b's A at 3BSD + b*S*S, A[i][j] at j + S*i
    A = host(cache)[3 * B * S * D:3 * B * S * D + B * S * S].reshape(B, S, S)
    ok, msg = close(A, from_cm(r_attn, (B, S, S)), 1e-4, 1e-5)
    assert ok, f"attn: {msg}"
    checks = [(host(out), r_out, cm(mags["out"]), "out"), (host(dX), r_dX, cm(mags["dX"]), "dX")]
    checks += [(host(g), r, cm(mags[n]), n) for g, r, n in zip(gW, r_g, ("gWq", "gWk", "gWv", "gWo"))]
    for got, want, mag, name in checks:
        ok, msg = close_mag(got, want, mag, 1e-4, 1e-5)
        assert ok, f"{name}: {msg}"
    # skip connections fused into the last GEMMs: equal to the separate adds
    out_r = torch.empty(B * S * D, device="cuda")
    cache_r = torch.empty_like(cache)
    ops.mha_forward_residual(*xd, *Wd, xd[0], out_r, cache_r, B, S, D, h)
    want_r = torch.empty(B * S * D, device="cuda")
    ops.add(out, xd[0], want_r)
    np.testing.assert_array_equal(host(out_r), host(want_r))
    skip = dev(cm(dy * 3))
    dX_r = torch.empty(B * S * D, device="cuda")
    gW_r = [torch.empty(D * D, device="cuda") for _ in range(4)]
    if self_attn:
        gall_r = torch.empty(4 * D * D, device="cuda")
        gW_r = [gall_r[i * D * D:(i + 1) * D * D] for i in range(4)]
    ops.mha_backward_residual(*xd, *Wd, cache_r, dev(cm(dy)), skip, *gW_r, dX_r, B, S, D, h)
    want_dx = torch.empty(B * S * D, device="cuda")
    ops.add(dX, skip, want_dx)
    np.testing.assert_array_equal(host(dX_r), host(want_dx))
    for a, b_ in zip(gW_r, gW):
        np.testing.assert_array_equal(host(a), host(b_))


def to_by_sample(flat, B, S, D):
    """ColMajor [B, S, D] (row b + B*s) -> rows s + S*b."""
    return np.ascontiguousarray(np.asarray(flat).reshape(D, S, B).transpose(0, 2, 1)).ravel()


def from_by_sample(flat, B, S, D):
    return np.ascontiguousarray(np.asarray(flat).reshape(D, B, S).transpose(0, 2, 1)).ravel()


@pytest.mark.parametrize("self_attn", [True, False])
@pytest.mark.parametrize("B,S,D,h", MHA_CASES + [(3, 6, 8, 2)])
def test_mha_by_sample_rows(gpu, B, S, D, h, self_attn):
    """The by-sample row order (no transposes) against the reference order on
    the same data: every row-wise result (output, attention weights, dX) is
    bit-identical, since each element is the same sum in the same order; the
    weight gradients, sums over all B*S rows taken in another row order, are
    within the per-element contraction bar."""
    print(f"[mha rows] B={B} S={S} D={D} heads={h} self={self_attn}", flush=True)
    rng = np.random.default_rng(B * 5 + S + D + self_attn)
    lim = np.sqrt(6.0 / (2 * D))
    Ws = [rng.uniform(-lim, lim, (D, D)).astype(np.float32) for _ in range(4)]
    xs = [rng.standard_normal((B, S, D)).astype(np.float32) for _ in range(1 if self_attn else 3)]
    if self_attn:
        xs = xs * 3
    dy = (rng.standard_normal((B, S, D)) * 1e-2).astype(np.float32)
    skip = (rng.standard_normal((B, S, D)) * 1e-2).astype(np.float32)
    Wc = np.concatenate([cm(w) for w in Ws])
    runs = {}
    for rows in (ops.ROWS_REF, ops.ROWS_BY_SAMPLE):
        order = (lambda a: a) if rows == ops.ROWS_REF else (lambda a: to_by_sample(a, B, S, D))
        Wall = dev(Wc)
        Wd = [Wall[i * D * D:(i + 1) * D * D] for i in range(4)]
        gall = torch.full((4 * D * D,), 7.0, device="cuda")
        gW = [gall[i * D * D:(i + 1) * D * D] for i in range(4)]
        xd = [dev(order(cm(x))) for x in xs]
        if self_attn:
            xd = [xd[0]] * 3
        out = torch.empty(B * S * D, device="cuda")
        cache = torch.empty(ops.mha_cache_floats(B, S, D), device="cuda")
        ops.mha_forward_residual(*xd, *Wd, xd[0], out, cache, B, S, D, h, rows=rows)
        dX = torch.empty(B * S * D, device="cuda")
        ops.mha_backward_residual(*xd, *Wd, cache, dev(order(cm(dy))), dev(order(cm(skip))), *gW, dX,
                                  B, S, D, h, rows=rows)
        back = (lambda a: a) if rows == ops.ROWS_REF else (lambda a: from_by_sample(a, B, S, D))
        A = host(cache)[3 * B * S * D:3 * B * S * D + B * S * S]
        runs[rows] = (back(host(out)), A, back(host(dX)), [host(g) for g in gW])
    ref, bys = runs[ops.ROWS_REF], runs[ops.ROWS_BY_SAMPLE]
    for k, name in enumerate(("out", "attention weights", "dX")):
        np.testing.assert_array_equal(bys[k], ref[k], err_msg=name)
    mags = _mha_logical([x.astype(np.float64) for x in xs], [w.astype(np.float64) for w in Ws],
                        dy.astype(np.float64), h)
    for got, want, n in zip(bys[3], ref[3], ("gWq", "gWk", "gWv", "gWo")):
        ok, msg = close_mag(got, want, cm(mags[n]), 1e-4, 1e-5)
        assert ok, f"{n}: {msg}"


def test_mha_rejects_bad_heads(gpu):
    from cppnet_amd import _capi
    x = torch.zeros(2 * 3 * 6, device="cuda")
    w = torch.zeros(36, device="cuda")
    cache = torch.empty(ops.mha_cache_floats(2, 3, 6), device="cuda")
    with pytest.raises(_capi.CnhipError, match="heads"):
        ops.mha_forward(x, x, x, w, w, w, w, x.clone(), cache, 2, 3, 6, 4)


# ---------------------------------------------------------------- embedding
# up to 8192 tokens over up to 8192 ids the backward buckets the tokens in one
# block (config 5's 32 x 256 over 8192 is one such; 64 x 128 over 300 ids puts
# ~27 tokens in each bucket); 40 x 256 over 9000 ids takes the multi-launch path
@pytest.mark.parametrize("B,S,V,D", [(3, 5, 7, 4), (4, 33, 50, 70), (32, 256, 8192, 512), (64, 128, 300, 16),
                                     (40, 256, 9000, 8)])
def test_embedding_exact(gpu, oracle, B, S, V, D):
    print(f"[embedding] B={B} S={S} V={V} D={D}", flush=True)
    rng = np.random.default_rng(B + S + V + D)
    ids = rng.integers(0, V, (B, S)).astype(np.int32)
    ids[0, : min(S, 3)] = 1  # repeated ids accumulate
    ids[-1, -1] = V - 1
    W = rng.uniform(-1 / np.sqrt(D), 1 / np.sqrt(D), (V, D)).astype(np.float32)
    dy = rng.standard_normal((B, S, D)).astype(np.float32)
    idc = cm(ids).astype(np.int32)
    Wt = np.ascontiguousarray(W).ravel()  # token-major: Wt[d + D*v] = W[v, d]
    out = torch.empty(B * S * D, device="cuda")
    oob = torch.zeros(1, dtype=torch.int32, device="cuda")
    ops.embedding_forward(dev(idc), dev(Wt), out, B, S, V, D, oob)
    r_out = np.zeros(B * S * D, np.float32)
    assert oracle.cnref_embedding_forward(ip(idc), fp(cm(W)), fp(r_out), B, S, V, D) == 0
    np.testing.assert_array_equal(host(out), r_out)
    assert int(host(oob)[0]) == 0
    gWt = torch.full((V * D,), 3.0, device="cuda")
    ops.embedding_backward(dev(idc), dev(cm(dy)), gWt, B, S, V, D)
    r_g = np.zeros(V * D, np.float32)
    oracle.cnref_embedding_backward(ip(idc), fp(cm(dy)), fp(r_g), B, S, V, D)
    np.testing.assert_array_equal(host(gWt).reshape(V, D), from_cm(r_g, (V, D)))
    # by sample: the same rows at s + S*b, and the same per-token sums in the same order
    ops.embedding_forward(dev(idc), dev(Wt), out, B, S, V, D, oob, rows=ops.ROWS_BY_SAMPLE)
    np.testing.assert_array_equal(host(out), to_by_sample(r_out, B, S, D))
    gWt.fill_(3.0)
    ops.embedding_backward(dev(idc), dev(to_by_sample(cm(dy), B, S, D)), gWt, B, S, V, D,
                           rows=ops.ROWS_BY_SAMPLE)
    np.testing.assert_array_equal(host(gWt).reshape(V, D), from_cm(r_g, (V, D)))


def test_embedding_out_of_range_ids_counted(gpu):
    B, S, V, D = 2, 3, 5, 4
    ids = np.array([[0, 5, 2], [-1, 4, 1]], np.int32)
    W = np.arange(V * D, dtype=np.float32).reshape(V, D) + 1
    out = torch.empty(B * S * D, device="cuda")
    oob = torch.zeros(1, dtype=torch.int32, device="cuda")
    ops.embedding_forward(dev(cm(ids)), dev(W.ravel()), out, B, S, V, D, oob)
    assert int(host(oob)[0]) == 2
    got = from_cm(host(out), (B, S, D))
    assert not got[0, 1].any() and not got[1, 0].any()
    np.testing.assert_array_equal(got[1, 1], W[4])


# ---------------------------------------------------------------- BatchNorm
@pytest.mark.parametrize("N,F", [(64, 6), (1000, 3), (8192, 512), (9000, 5), (1001, 3), (40000, 2)])
def test_batchnorm_vs_oracle(gpu, oracle, N, F):
    print(f"[batchnorm] N={N} F={F}", flush=True)
    rng = np.random.default_rng(N + F)
    x = (rng.standard_normal(N * F) * 2 + 0.5).astype(np.float32)
    gamma = (1 + 0.2 * rng.standard_normal(F)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(F)).astype(np.float32)
    rm0, rv0 = (0.1 * rng.standard_normal(F)).astype(np.float32), np.ones(F, np.float32)
    dy = rng.standard_normal(N * F).astype(np.float32)
    y, xh = torch.empty(N * F, device="cuda"), torch.empty(N * F, device="cuda")
    rm, rv = dev(rm0.copy()), dev(rv0.copy())
    bm, bv = torch.empty(F, device="cuda"), torch.empty(F, device="cuda")
    ops.batchnorm_forward(dev(x), y, xh, dev(gamma), dev(beta), rm, rv, bm, bv, N, F, 0.1, 1e-5)
    gg, gb, dX = torch.empty(F, device="cuda"), torch.empty(F, device="cuda"), torch.empty(N * F, device="cuda")
    ops.batchnorm_backward(dev(dy), dev(x), xh, dev(gamma), bm, bv, gg, gb, dX, N, F, 1e-5)
    r = {k: np.zeros(N * F, np.float32) for k in ("y", "xh", "dX")}
    r.update({k: np.zeros(F, np.float32) for k in ("bm", "bv", "gg", "gb")})
    rrm, rrv = rm0.copy(), rv0.copy()
    oracle.cnref_batchnorm_forward(fp(x), fp(r["y"]), fp(r["xh"]), fp(gamma), fp(beta), fp(rrm),
                                   fp(rrv), fp(r["bm"]), fp(r["bv"]), N, F, 0.1, 1e-5)
    oracle.cnref_batchnorm_backward(fp(dy), fp(x), fp(r["xh"]), fp(gamma), fp(r["bm"]), fp(r["bv"]),
                                    fp(r["gg"]), fp(r["gb"]), fp(r["dX"]), N, F, 1e-5)
    for got, want, name in [(host(y), r["y"], "y"), (host(xh), r["xh"], "xhat"), (host(bm), r["bm"], "mean"),
                            (host(bv), r["bv"], "var"), (host(rm), rrm, "running_mean"),
                            (host(rv), rrv, "running_var")]:
        ok, msg = close(got, want, 1e-4, 1e-5)
        assert ok, f"{name}: {msg}"
    # grads: sums over N; dX cancels three terms of size |g dy| / std
    xhat = r["xh"].reshape(F, N)
    ady = np.abs(dy.reshape(F, N)).astype(np.float64)
    inv_std = 1 / np.sqrt(r["bv"].astype(np.float64) + 1e-5)
    m_gg = (ady * np.abs(xhat)).sum(1) / np.sqrt(N)
    m_gb = ady.sum(1) / np.sqrt(N)
    term = (np.abs(gamma) * inv_std)[:, None]
    m_dx = term * (ady + (ady * np.abs(xhat)).sum(1, keepdims=True) * np.abs(xhat) / N
                   + ady.sum(1, keepdims=True) / N)
    for got, want, mag, name in [(host(gg), r["gg"], m_gg, "grad_gamma"), (host(gb), r["gb"], m_gb, "grad_beta"),
                                 (host(dX), r["dX"], m_dx.ravel(), "dX")]:
        ok, msg = close_mag(got, want, mag, 1e-4, 1e-5)
        assert ok, f"{name}: {msg}"
    # without xhat: the forward does not store it and the backward recomputes
    # it with the forward's expression -- the same bits everywhere
    y2, rm2, rv2 = torch.empty(N * F, device="cuda"), dev(rm0.copy()), dev(rv0.copy())
    bm2, bv2 = torch.empty(F, device="cuda"), torch.empty(F, device="cuda")
    ops.batchnorm_forward(dev(x), y2, None, dev(gamma), dev(beta), rm2, rv2, bm2, bv2, N, F, 0.1, 1e-5)
    gg2, gb2, dX2 = torch.empty(F, device="cuda"), torch.empty(F, device="cuda"), torch.empty(N * F, device="cuda")
    ops.batchnorm_backward(dev(dy), dev(x), None, dev(gamma), bm2, bv2, gg2, gb2, dX2, N, F, 1e-5)
    for a, b, name in [(y2, y, "y"), (bm2, bm, "mean"), (bv2, bv, "var"), (rm2, rm, "running_mean"),
                       (rv2, rv, "running_var"), (gg2, gg, "grad_gamma"), (gb2, gb, "grad_beta"), (dX2, dX, "dX")]:
        assert np.array_equal(host(a).view(np.uint32), host(b).view(np.uint32)), f"{name} differs without xhat"


# ---------------------------------------------------------------- GELU / pool / add
def test_gelu_vs_oracle(gpu, oracle):
    x = np.concatenate([np.linspace(-12, 12, 100001), np.random.default_rng(5).standard_normal(1 << 20) * 3])
    x = x.astype(np.float32)
    dy = np.cos(x).astype(np.float32)
    y, dx = torch.empty(x.size, device="cuda"), torch.empty(x.size, device="cuda")
    ops.gelu_forward(dev(x), y)
    ops.gelu_backward(dev(x), dev(dy), dx)
    ry, rdx = np.zeros_like(x), np.zeros_like(x)
    oracle.cnref_gelu_forward(fp(x), fp(ry), x.size)
    oracle.cnref_gelu_backward(fp(x), fp(dy), fp(rdx), x.size)
    for got, want, name in [(host(y), ry, "y"), (host(dx), rdx, "dx")]:
        ok, msg = close(got, want, 1e-5, 1e-7)
        assert ok, f"{name}: {msg}"
    # pointers off 16-byte alignment take the scalar path: same values
    xd, dyd = dev(x), dev(dy)
    y1, dx1 = torch.empty(x.size, device="cuda"), torch.empty(x.size, device="cuda")
    ops.gelu_forward(xd[1:], y1[1:])
    ops.gelu_backward(xd[1:], dyd[1:], dx1[1:])
    np.testing.assert_array_equal(host(y1)[1:], host(y)[1:])
    np.testing.assert_array_equal(host(dx1)[1:], host(dx)[1:])


@pytest.mark.parametrize("B,S,D", [(3, 7, 5), (32, 256, 512), (1, 1, 1), (100, 33, 6), (7, 1000, 3)])
def test_meanpool1d_vs_oracle(gpu, oracle, B, S, D):
    rng = np.random.default_rng(B + S + D)
    x, dy = rng.standard_normal(B * S * D).astype(np.float32), rng.standard_normal(B * D).astype(np.float32)
    y, dx = torch.empty(B * D, device="cuda"), torch.empty(B * S * D, device="cuda")
    ops.meanpool1d_forward(dev(x), y, B, S, D)
    ops.meanpool1d_backward(dev(dy), dx, B, S, D)
    ry, rdx = np.zeros(B * D, np.float32), np.zeros(B * S * D, np.float32)
    oracle.cnref_meanpool1d_forward(fp(x), fp(ry), B, S, D)
    oracle.cnref_meanpool1d_backward(fp(dy), fp(rdx), B, S, D)
    # forward sums s in chunks combined in a fixed order (the oracle sums
    # sequentially): fp32 rounding of a length-S sum, relative to the RMS size
    ok, msg = close_mag(host(y), ry, np.full(ry.shape, np.sqrt(np.mean(x.astype(np.float64) ** 2))), 1e-5, 1e-7)
    assert ok, msg
    np.testing.assert_array_equal(host(dx), rdx)
    # by sample (rows s + S*b): lane-strided partial sums, the same bar; the broadcast exact
    ops.meanpool1d_forward(dev(to_by_sample(x, B, S, D)), y, B, S, D, rows=ops.ROWS_BY_SAMPLE)
    ops.meanpool1d_backward(dev(dy), dx, B, S, D, rows=ops.ROWS_BY_SAMPLE)
    ok, msg = close_mag(host(y), ry, np.full(ry.shape, np.sqrt(np.mean(x.astype(np.float64) ** 2))), 1e-5, 1e-7)
    assert ok, f"by sample: {msg}"
    np.testing.assert_array_equal(host(dx), to_by_sample(rdx, B, S, D))


@pytest.mark.parametrize("n", [1, 7, 4096, 8192 * 512 + 3])
def test_add_exact(gpu, n):
    rng = np.random.default_rng(n)
    a, b = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    y = torch.empty(n, device="cuda")
    ops.add(dev(a), dev(b), y)
    np.testing.assert_array_equal(host(y), a + b)
