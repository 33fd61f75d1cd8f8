"""100 training steps at full layer widths, every config but C1 (whose
full-size 100-step run is in test_gpu_model.py), a fresh batch every step:

  C2  MLP 1024-4096-4096-10, batch 256
  C3  CNN 3->32->64 (3x3, pool 2) -> 4096->10, batch 128
  C4  LSTM 128->512, T 64 -> 512->1, batch 32
  C5  Embedding 8192x512, 2 x [MHA(512, 8) + BN + FFN 2048], S 256, batch 4

The gate is re-anchored every step (within rel 1e-4 /
abs 1e-5 after a step, within rel 1e-3 after 100).  Before each of the 100
steps the oracle is loaded with the GPU session's current parameters and
its Adam state (m, v and each parameter's step count t, adam.cpp:98-133),
runs one step on the same batch, and the GPU's step is held to the one-step
bars:
* the loss within rel 1e-4 / abs 1e-5;
* every gradient within 1e-5 + 1e-4 max(|ref|, mag), mag the per-element
  size (|A|^T|B|)/sqrt(R) of its contraction over R rows (a cancelled fp32
  sum carries ~u sqrt(R) of it on any evaluation order); for the MLP and
  the CNN plus the allowances for ReLU masks at near-zero pre-activations
  and near-tied max-pool windows (tests/model_bars.py), which may cover at
  most 1 in 10^3 of a layer's routing decisions (a mask flip moves a whole
  column of the weight gradient, so what is counted is the decisions);
  where an entry still misses, it is held instead to the oracle run with
  double accumulation (rounded once per element, the closest of its orders
  to exact) within the bar plus twice the largest distance from that run of
  the oracle's fp32 orders (its own and three others), all one step from
  the same state.  The contraction bar bounds one contraction's rounding;
  an embedding row of a token seen once is the end of the whole backward
  chain, whose rounding it does not bound.  (On RMS over each tensor the
  GPU's gradients are closer to the double-accumulated oracle than the fp32
  oracle is, 0.2-1.2x its distance; per element, two independent fp32
  roundings meet in the tails of a 4 M-entry tensor.);
* Adam's m and v within what that gradient bar allows through their update
  ((1-b1) dg, (1-b2)(2|g| + dg) dg) plus 1e-6 relative rounding, and the
  same step counts;
* the updated parameters within 1e-5 + 1e-4 |ref|, except where Adam's
  update itself is that sensitive to the gradient: there the bound is the
  largest change of lr mhat / (sqrt(vhat) + eps) over gradients within the
  gradient bar (float64, five points of the interval), which is what lets a
  near-zero gradient's sign flip a first step by ~2 lr.
Each step's worst ratio of error to bar is reported per config.

The same 100 steps are also run by a free-running oracle (never re-anchored)
and its distance from the GPU printed -- a report, not a gate: at these
batches C3 and C5 are chaotic under Adam (the oracle's own valid fp32
evaluation orders part by 10-200% within 100 steps), so a free-running
comparison cannot tell a correct GPU from a wrong one there.

With CNT_PARITY_REPORT set to a path, each run appends its progress and
results there as JSON lines."""
import json
import os
import time
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from cppnet_amd import trainer
from contraction_mags import rnn_mags, transformer_mags
from model_bars import _cnn_mags, _cnn_tie_allowance, _grad_mags, _mask_allowance

pytestmark = pytest.mark.gpu

STEPS = 100


def _runs():
    from oracle.cnn import OracleCNN
    from oracle.mlp import OracleMLP
    from oracle.rnn import OracleSeqRegressor
    from oracle.transformer import OracleTransformer
    return {
        "C2": (lambda: trainer.mlp_config(2, 256), trainer.synthetic_mlp, OracleMLP, "mlp"),
        "C3": (lambda: trainer.cnn_config(3, 128), trainer.synthetic_cnn, OracleCNN, "cnn"),
        "C4": (lambda: trainer.rnn_config(4, batch=32), trainer.synthetic_rnn, OracleSeqRegressor, "rnn"),
        "C5": (lambda: trainer.transformer_config(5, batch=4), trainer.synthetic_transformer,
               OracleTransformer, "transformer"),
    }


@pytest.fixture(scope="module")
def oracle_mt(oracle):
    oracle.cnref_set_threads(min(16, os.cpu_count() or 1))
    return oracle


def _report(**rec):
    path = os.environ.get("CNT_PARITY_REPORT")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(rec) + "\n")
    print(json.dumps(rec), flush=True)


def _rel(a, b):
    return float(np.linalg.norm(a.astype(np.float64) - b) / max(np.linalg.norm(b), 1e-30))


def _anchor(ref, params, m, v, t):
    """The oracle model at the GPU's parameters and Adam state (copied into
    its arrays in place after the first call: each step zeroes or overwrites
    its gradients itself)."""
    if getattr(ref, "params", None) is None:
        ref.set_params(params)
    st = ref.opt if hasattr(ref, "opt") else ref  # MLP / RNN keep theirs in an OracleOptimizer
    for dst, src in zip(ref.params + st.m + st.v, list(params) + list(m) + list(v)):
        np.copyto(dst, src)
    st.t = list(t)


def _bars(kind, oracle, ref, cfg, params, stats):
    """(per-gradient magnitudes, lazy allowance function); the allowance
    function appends to stats, per layer, (routing decisions rounding may
    take either way, decisions)."""
    if kind == "mlp":
        return _grad_mags(oracle, ref, cfg), lambda: _mask_allowance(oracle, ref, cfg, params, stats)
    if kind == "cnn":
        return _cnn_mags(oracle, ref, cfg), lambda: _cnn_tie_allowance(oracle, ref, cfg, params, stats)
    if kind == "rnn":
        return rnn_mags(oracle, ref, cfg), None
    return transformer_mags(oracle, ref, cfg, params), None


def _adam_update(w, m, v, g, bc1, bc2, cfg):
    """W - lr mhat / (sqrt(vhat) + eps) in float64 for gradient g (adam.cpp:121-130)."""
    m1 = cfg.beta1 * m + (1.0 - cfg.beta1) * g
    v1 = cfg.beta2 * v + (1.0 - cfg.beta2) * g * g
    return w - cfg.lr * (m1 / bc1) / (np.sqrt(v1 / bc2) + cfg.eps)


_POOL = ThreadPoolExecutor(max(1, min(16, os.cpu_count() or 1)))


def _chunked(fn, n, size=1 << 19):
    """fn(slice) over n elements in chunks on the thread pool (numpy's
    elementwise loops release the GIL)."""
    return list(_POOL.map(fn, [slice(s, min(n, s + size)) for s in range(0, n, size)]))


def _tensor_ratios(a, b, mag, al, mo, vo, mg, vg, wo, wg, b1, b2, gref=None):
    """Per-element checks of one parameter's gradient a (oracle b; compared
    with gref when given), Adam moments mg, vg (oracle mo, vo) and updated
    value wg (oracle wo), chunked: (entries over the gradient bar, worst
    gradient / m / v ratios, worst ratio within the strict bar of the
    updated values, indices of those beyond it)."""
    gref = b if gref is None else gref

    def run(sl):
        lim = np.maximum(np.abs(b[sl]), mag[sl])
        lim *= 1e-4
        lim += 1e-5
        if al is not None:
            lim += al[sl]
        err = np.subtract(a[sl], gref[sl])
        np.abs(err, out=err)
        over = int(np.count_nonzero(err > lim))
        np.divide(err, lim, out=err)
        rg = float(err.max())
        # Adam's moments: the gradient's bar carried through their update
        # (1.001x for the float32 evaluation of the bar itself)
        bar = np.abs(mo[sl])
        bar *= 1e-6
        bar += np.float32((1.0 - b1) * 1.001) * lim
        bar += np.float32(1e-30)
        d = np.subtract(mg[sl], mo[sl])
        np.abs(d, out=d)
        np.divide(d, bar, out=d)
        rm = float(d.max())
        bar = np.abs(b[sl])
        bar *= 2.0
        bar += lim
        bar *= lim
        bar *= np.float32((1.0 - b2) * 1.001)
        bar += np.float32(1e-6) * np.abs(vo[sl])
        bar += np.float32(1e-30)
        np.subtract(vg[sl], vo[sl], out=d)
        np.abs(d, out=d)
        np.divide(d, bar, out=d)
        rv = float(d.max())
        strict = np.abs(wo[sl])
        strict *= 1e-4
        strict += 1e-5
        np.subtract(wg[sl], wo[sl], out=d)
        np.abs(d, out=d)
        np.divide(d, strict, out=d)  # the ratio to the strict bar
        bad = np.nonzero(d > 1.0)[0]
        rp = float(d.max())
        if bad.size:  # the largest ratio among the elements within the strict bar
            d[bad] = 0.0
            rp = float(d.max())
        return over, rg, rm, rv, rp, bad + sl.start
    parts = _chunked(run, a.size)
    return (sum(p[0] for p in parts), max(p[1] for p in parts), max(p[2] for p in parts),
            max(p[3] for p in parts), max(p[4] for p in parts), np.concatenate([p[5] for p in parts]))


# (double accumulation, fp32 sum order) of the oracle's other valid
# evaluation orders: double accumulation rounded once per element; fp32
# descending; fp32 in 32-wide chunks summed in order; fp32 in 8 strided
# partial sums combined pairwise (GEMM k-sums, bias column sums, conv weight
# and bias sums, BatchNorm and mean-pool sums)
ORDERS = [(1, 0), (0, 1), (0, 2), (0, 3)]


def _order_spread(alt, oracle, ref, state, X, Y):
    """The oracle's gradient with double accumulation (rounded once per
    element: the closest of its orders to exact) and, per element, the
    largest distance from it of the fp32 orders (the main oracle's and three
    others), each run one step from the same (GPU) state -- computed once
    per step, only when a gradient misses its bar."""
    cache = []

    def fn():
        if not cache:
            runs = []
            for double, order in ORDERS:
                _anchor(alt, *state)
                oracle.cnref_set_accumulate_double(double)
                oracle.cnref_set_sum_order(order)
                try:
                    alt.step(X, Y)
                finally:
                    oracle.cnref_set_accumulate_double(0)
                    oracle.cnref_set_sum_order(0)
                runs.append([g.copy() for g in alt.last_grads])
            fn.grads = runs
            dbl = runs[0]
            spread = [np.abs(r - d) for r, d in zip(ref.last_grads, dbl)]
            for other in runs[1:]:
                spread = [np.maximum(sp, np.abs(g - d)) for sp, g, d in zip(spread, other, dbl)]
            cache.append((dbl, spread))
        return cache[0]
    fn.grads = []  # each order's gradients, for the failure report
    return fn


def _check_step(name, k, cfg, oracle, ref, kind, params, m0, v0, t0, got, spread_fn):
    """One re-anchored step: the GPU's loss, gradients, m, v, t and updated
    parameters (`got`) against the oracle's from the same state.  A gradient
    entry beyond the contraction bar may use, in turn, the rounding-routing
    allowance (MLP, CNN) and then the double-accumulated oracle with twice
    the spread of the fp32 orders around it, from the same state
    (spread_fn).  Returns the step's
    worst error-to-bar ratios and how often each allowance was needed."""
    loss_g, grads_g, params_g, m_g, v_g, t_g = got
    loss_o = ref.loss
    out = {"loss": abs(loss_g - loss_o) / (1e-5 + 1e-4 * abs(loss_o)), "grad": 0.0, "m": 0.0, "v": 0.0,
           "param": 0.0, "allowance_used": 0, "order_spread_used": 0, "adam_bound_used": 0}
    assert out["loss"] <= 1.0, f"{name} step {k}: loss {loss_g!r} vs oracle {loss_o!r}"
    stats = []
    mags, allow_fn = _bars(kind, oracle, ref, cfg, params, stats)
    allow = None
    st = ref.opt if hasattr(ref, "opt") else ref
    assert list(t_g) == list(st.t), f"{name} step {k}: Adam step counts {t_g} vs {st.t}"
    b1, b2 = cfg.beta1, cfg.beta2
    for i, (a, b, mag) in enumerate(zip(grads_g, ref.last_grads, mags)):
        args = (st.m[i], st.v[i], m_g[i], v_g[i], ref.params[i], params_g[i], b1, b2)
        over, rg, rm, rv, rp, bad = _tensor_ratios(a, b, mag, None, *args)
        extra = None
        if over and allow_fn is not None:
            if allow is None:
                allow = allow_fn()
                # the allowance is nonzero only where a routing decision is
                # ambiguous; those must stay rare (a flipped ReLU mask moves a
                # whole column of the weight gradient, so the entries it
                # rescues are not a measure of how many decisions it covers)
                for layer, (n_amb, n_all) in enumerate(stats):
                    assert n_amb <= max(1, n_all // 1000), (
                        f"{name} step {k}: layer {layer}: {n_amb}/{n_all} routing decisions within rounding "
                        f"of a tie")
                out["ambiguous_decisions"] = out.get("ambiguous_decisions", 0) + sum(n for n, _ in stats)
            extra = allow[i] if allow[i].size == a.size else np.zeros_like(a)
            out["allowance_used"] += over
            over, rg, rm, rv, rp, bad = _tensor_ratios(a, b, mag, extra, *args)
        if over:
            # against the double-accumulated oracle, within the bar plus twice
            # the farthest fp32 order's distance from it; m, v and the updated
            # values (the fp32 oracle's) then within that plus their own distance
            dbl, spread = spread_fn()
            out["order_spread_used"] += over
            base = np.zeros_like(a) if extra is None else extra
            over, rg, _, _, _, _ = _tensor_ratios(a, b, mag, base + 2.0 * spread[i], *args, gref=dbl[i])
            if rg > 1.0:
                lim = 1e-5 + 1e-4 * np.maximum(np.abs(b), mag) + base + 2.0 * spread[i]
                j = int(np.argmax(np.abs(a - dbl[i]) / lim))
                detail = dict(index=j, got=float(a[j]), fp32=float(b[j]), mag=float(mag[j]),
                              farthest_fp32_order_from_double=float(spread[i][j]),
                              err_vs_double=float(abs(a[j] - dbl[i][j])))
                for alt_name, g_alt in zip(ORDERS, spread_fn.grads):
                    detail[f"order{alt_name}"] = float(g_alt[i][j])
                print(f"[long] {name} step {k} grad {i} worst entry: {json.dumps(detail)}", flush=True)
            assert rg <= 1.0, (f"{name} step {k}: grad {i}: {over}/{a.size} beyond the bar, the rounding-"
                               f"routing allowance and twice the oracle's own order spread ({rg:.3g}x)")
            extra = base + 3.0 * spread[i]
            _, _, rm, rv, rp, bad = _tensor_ratios(a, b, mag, extra, *args)
        out["grad"], out["m"], out["v"] = max(out["grad"], rg), max(out["m"], rm), max(out["v"], rv)
        assert rm <= 1.0, f"{name} step {k}: Adam m of param {i} beyond its bar ({rm:.3g}x)"
        assert rv <= 1.0, f"{name} step {k}: Adam v of param {i} beyond its bar ({rv:.3g}x)"
        if bad.size:
            # beyond 1e-5 + 1e-4 |ref|: the bound is Adam's own sensitivity to
            # a gradient within its bar
            bc1 = float(oracle.cnref_bias_correction(b1, st.t[i]))
            bc2 = float(oracle.cnref_bias_correction(b2, st.t[i]))
            w0 = params[i][bad].astype(np.float64)
            mm, vv = m0[i][bad].astype(np.float64), v0[i][bad].astype(np.float64)
            g = b[bad].astype(np.float64)
            gd = 1e-5 + 1e-4 * np.maximum(np.abs(g), mag[bad]) + (extra[bad] if extra is not None else 0.0)
            base = _adam_update(w0, mm, vv, g, bc1, bc2, cfg)
            spread = np.zeros_like(base)
            for f in (-1.0, -0.5, 0.5, 1.0):
                spread = np.maximum(spread, np.abs(_adam_update(w0, mm, vv, g + f * gd, bc1, bc2, cfg) - base))
            wo = ref.params[i][bad].astype(np.float64)
            e = np.abs(params_g[i][bad].astype(np.float64) - wo)
            r = e / (1e-5 + 1e-4 * np.abs(wo) + spread * 1.01)
            assert r.max() <= 1.0, (f"{name} step {k}: param {i}: {int((r > 1).sum())} updated weights beyond "
                                    f"the bar and Adam's sensitivity to the gradient bar (worst {float(r.max()):.3g}x)")
            rp = max(rp, float(r.max()))
            out["adam_bound_used"] += int(bad.size)
        out["param"] = max(out["param"], rp)
    return out


@pytest.mark.parametrize("name", ["C2", "C3", "C4", "C5"])
def test_100_steps_full_width_reanchored(gpu, oracle_mt, name):
    make, synth, Ref, kind = _runs()[name]
    cfg = make()
    print(f"[long] {name} batch {cfg.batch}: {STEPS} re-anchored steps", flush=True)
    seed = 900 + int(name[1])
    params = synth(cfg, np.random.default_rng(seed))[0]
    sess = trainer.Session(cfg)
    sess.set_params(params)
    ref = Ref(cfg, oracle_mt)           # re-anchored to the GPU every step: the gate
    alt = Ref(cfg, oracle_mt)           # the same step under the oracle's other orders, when needed
    free = Ref(cfg, oracle_mt)          # never re-anchored: the report
    free.keep = False
    free.set_params(params)
    brng = np.random.default_rng(seed + 1)
    t0 = time.time()
    cur = [np.array(p, np.float32) for p in params]
    m_cur, v_cur = [np.zeros_like(p) for p in cur], [np.zeros_like(p) for p in cur]
    t_cur = [0] * len(cur)
    worst = {}
    lg, lf = np.zeros(STEPS), np.zeros(STEPS)
    for step in range(STEPS):
        X, Y = trainer.synthetic_batch(cfg, brng)
        _anchor(ref, cur, m_cur, v_cur, t_cur)
        ref.loss = ref.step(X, Y)
        sess.set_batch(X, Y)
        loss_g = sess.forward_backward()
        grads_g = sess.get_grads()
        sess.update()
        new = sess.get_params()
        m_new, t_new = sess.get_opt_state(0)
        v_new, _ = sess.get_opt_state(1)
        res = _check_step(name, step, cfg, oracle_mt, ref, kind, cur, m_cur, v_cur, t_cur,
                          (loss_g, grads_g, new, m_new, v_new, t_new),
                          _order_spread(alt, oracle_mt, ref, (cur, m_cur, v_cur, t_cur), X, Y))
        for key, val in res.items():
            counted = key in ("allowance_used", "order_spread_used", "adam_bound_used", "ambiguous_decisions")
            worst[key] = worst.get(key, 0) + val if counted else max(worst.get(key, 0), val)
        cur, m_cur, v_cur, t_cur = new, m_new, v_new, t_new
        lg[step], lf[step] = loss_g, free.step(X, Y)
        if step % 10 == 9:
            _report(config=name, step=step + 1, loss_gpu=float(loss_g), worst_ratio_so_far=worst,
                    seconds=round(time.time() - t0, 1))
    sess.close()
    free_rel = [_rel(a, b) for a, b in zip(cur, free.get_params())]
    _report(config=name, batch=cfg.batch, steps=STEPS, reanchored_worst_ratio=worst,
            free_running_report=dict(worst_loss_rel=float((np.abs(lg - lf) / np.abs(lf)).max()),
                                     first_step_loss_rel_over_1e3=(int(np.argmax(np.abs(lg - lf) > 1e-3 * np.abs(lf)))
                                                                   if (np.abs(lg - lf) > 1e-3 * np.abs(lf)).any()
                                                                   else None),
                                     param_rel_after=[round(r, 6) for r in free_rel]),
            seconds=round(time.time() - t0, 1))
