"""Error bars of the model-level parity tests (test infrastructure): the
per-element magnitudes of each parameter gradient's contraction and the
allowances for rounding-level routing decisions (ReLU masks at near-zero
pre-activations, near-tied max-pool windows), computed from the oracle's own
traced operands (oracle/mlp.py, oracle/cnn.py)."""
import numpy as np

from oracle_lib import fp, gemm_mag


def _grad_mags(oracle, ref, cfg):
    """Per-element magnitude (|X|^T|dA|)/sqrt(B) of each W grad, and the bias
    analogue, from the oracle's own layer inputs and pre-activation grads."""
    mags = []
    B = cfg.batch
    for i, tr in enumerate(ref.trace):
        I, O = cfg.sizes[i], cfg.sizes[i + 1]
        mags.append(gemm_mag(oracle, 1, 0, I, O, B, tr["x"], B, tr["dA"], B, I))
        mags.append(gemm_mag(oracle, 1, 0, 1, O, B, np.ones(B, np.float32), B, tr["dA"], B, 1))
    return mags


# activations with a kink at 0: the jump of the slope there (ReLU 1, LeakyReLU 1 - alpha)
_KINKED = {"relu": 1.0, "leaky_relu": 0.99}


def _mask_allowance(oracle, ref, cfg, params, stats=None):
    """Bound on what ReLU-mask choices at near-zero pre-activations can change.

    S_l = {(b,o): |z_l| <= tau_l} with tau_l the forward bound of z_l
    (1e-5 + 1e-4 max(|z|, (|x||W|)/sqrt(I)) + |b|-rounding).  Flipping mask
    entries of S_l changes dA_l by at most E_l = |dH_l| on S_l, and, through
    dX_l = dA_l W_l^T, changes dH_{l-1} by at most E_l |W_l|^T.  Each
    gradient's allowance is the contraction of |x_l| with the total change of
    dA_l (own flips + masked upstream change)."""
    B = cfg.batch
    nl = len(ref.trace)
    E = [None] * nl            # |change of dA_l| from flips at layer l, ColMajor [B,O_l]
    up = [None] * nl           # |change of dH_l| from flips at layer l+1
    for i, tr in enumerate(ref.trace):
        I, O = cfg.sizes[i], cfg.sizes[i + 1]
        if tr["act"] not in _KINKED:
            E[i] = np.zeros(B * O, np.float32)
            continue
        zmag = gemm_mag(oracle, 0, 0, B, O, I, tr["x"], B, params[2 * i], I, B)
        tau = 1e-5 + 1e-4 * np.maximum(np.abs(tr["z"]), zmag)
        amb = np.abs(tr["z"]) <= tau
        if stats is not None:  # pre-activations whose mask rounding may decide
            stats.append((int(amb.sum()), amb.size))
        E[i] = np.where(amb, _KINKED[tr["act"]] * np.abs(tr["dH"]), 0.0).astype(np.float32)
    allow = []
    for i, tr in enumerate(ref.trace):
        I, O = cfg.sizes[i], cfg.sizes[i + 1]
        dchg = E[i].copy()
        if i + 1 < nl:
            O2 = cfg.sizes[i + 2]
            d_up = np.zeros(B * O, np.float32)   # |E_{l+1}| |W_{l+1}|^T : [B, O]
            oracle.cnref_gemm_f32(0, 1, B, O, O2, 1.0, fp(E[i + 1]), B,
                                  fp(np.abs(params[2 * (i + 1)])), O, 0.0, fp(d_up), B, None, 0)
            mask = (np.where(tr["z"] > 0, 1.0, 1.0 - _KINKED[tr["act"]]).astype(np.float32)
                    if tr["act"] in _KINKED else 1.0)
            dchg = dchg + d_up * np.maximum(mask, (E[i] > 0))
        dchg = dchg.astype(np.float32)
        aW = np.zeros(I * O, np.float32)
        oracle.cnref_gemm_f32(1, 0, I, O, B, 1.0, fp(np.abs(tr["x"])), B, fp(dchg), B, 0.0,
                              fp(aW), I, None, 0)
        ab = np.zeros(O, np.float32)
        oracle.cnref_column_sum(fp(dchg), fp(ab), B, O, 0)
        allow += [aW, ab]
    return allow


def _cnn_mags(oracle, ref, cfg):
    """Per-gradient magnitudes: the same contractions over |inputs| / sqrt(len)."""
    from oracle import fp as _fp
    mags = []
    N = cfg.batch
    for tr in ref.trace:
        ic, oc, k, s, p, H, W, HO, WO = tr["dims"]
        mW, mb = np.zeros(oc * ic * k * k, np.float32), np.zeros(oc, np.float32)
        mdx = np.zeros(N * ic * H * W, np.float32)
        wabs = np.ones(oc * ic * k * k, np.float32)
        oracle.cnref_conv2d_backward(_fp(np.abs(tr["x"])), _fp(wabs), _fp(np.abs(tr["dz"])), _fp(mW),
                                     _fp(mb), _fp(mdx), N, ic, H, W, oc, k, s, p)
        L = np.sqrt(N * HO * WO)
        mags += [mW / L, mb / L]
    fc = ref.fc_trace
    mags.append(gemm_mag(oracle, 1, 0, fc["F"], cfg.classes, N, fc["x"], N, fc["g"], N, fc["F"]))
    mags.append(gemm_mag(oracle, 1, 0, 1, cfg.classes, N, np.ones(N, np.float32), N, fc["g"], N, 1))
    return mags


def _cm(flat, shape):
    """flat Eigen ColMajor buffer -> logical array of the given shape (a view)."""
    return np.asarray(flat).reshape(tuple(reversed(shape))).transpose(*reversed(range(len(shape))))


def _to_cm(arr):
    return np.ascontiguousarray(arr.transpose(*reversed(range(arr.ndim)))).ravel().astype(np.float32)


def _cnn_tie_allowance(oracle, ref, cfg, params, stats=None):
    """Bound on what rounding-level routing decisions can change in the conv
    gradients.  Per block (conv -> ReLU -> max-pool):
    * a ReLU input within forward tolerance tau of 0 may be gated either way,
      changing dz by |da| there;
    * a pool window whose runner-up lies within tau of its maximum may route
      its gradient g to any of the near-maximal positions, changing da by |g|
      at each of them;
    so dz may change by E (elementwise).  The conv backward of (|x|, |W|, E)
    bounds the change of dW, db and of the gradient handed to the block
    below, which is routed through that block's pool and ReLU in turn."""
    from oracle import fp as _fp
    N, pool = cfg.batch, cfg.pool
    allow = [None] * (2 * len(ref.trace))
    carry = None  # |change| of the gradient at this block's pool output
    for i in reversed(range(len(ref.trace))):
        tr = ref.trace[i]
        ic, oc, k, s, p, H, W, HO, WO = tr["dims"]
        Wt = params[2 * i]
        zmag = np.zeros(N * oc * HO * WO, np.float32)
        oracle.cnref_conv2d_forward(_fp(np.abs(tr["x"])), _fp(np.abs(Wt)), None, _fp(zmag), N, ic, H,
                                    W, oc, k, s, p)
        tau = 1e-5 + 1e-4 * np.maximum(np.abs(tr["z"]), zmag / np.sqrt(ic * k * k))
        relu_amb = np.abs(tr["z"]) <= tau
        PH, PW = (HO - pool) // pool + 1, (WO - pool) // pool + 1
        a = _cm(tr["a"], (N, oc, HO, WO))[:, :, :PH * pool, :PW * pool]
        t = _cm(tau, (N, oc, HO, WO))[:, :, :PH * pool, :PW * pool]
        win = a.reshape(N, oc, PH, pool, PW, pool)
        tw = t.reshape(N, oc, PH, pool, PW, pool)
        mx = win.max(axis=(3, 5), keepdims=True)
        tmx = tw.max(axis=(3, 5), keepdims=True)
        near = win >= mx - (tmx + tw)
        amb_win = near.sum(axis=(3, 5), keepdims=True) >= 2
        if stats is not None:
            # ReLU inputs within rounding of 0, and pool windows whose near-tied
            # maximum is a positive ReLU output (a window of zeros routes its
            # gradient to an input whose ReLU passes none of it)
            live = amb_win & (mx > tmx)
            stats.append((int(relu_amb.sum()) + int(live.sum()), relu_amb.size + amb_win.size))
        g = np.abs(_cm(tr["gpool"], (N, oc, PH, PW)))
        if carry is not None:
            g = g + _cm(carry, (N, oc, PH, PW))
        # change of da: |g| at every near-max position of an ambiguous window;
        # the upstream change (carry) lands on the argmax of every window
        da_chg = np.zeros((N, oc, HO, WO), np.float32)
        amb_part = np.where(near & amb_win, g[:, :, :, None, :, None], 0.0)
        da_chg[:, :, :PH * pool, :PW * pool] = amb_part.reshape(N, oc, PH * pool, PW * pool)
        if carry is not None:
            idx = _cm(tr["idx"], (N, oc, PH, PW))
            cflat = _cm(carry, (N, oc, PH, PW))
            for ph in range(pool):
                for pw in range(pool):
                    sel = idx == ph * pool + pw
                    da_chg[:, :, ph:PH * pool:pool, pw:PW * pool:pool] += np.where(sel, cflat, 0.0)
        da_chg = _to_cm(da_chg)
        gate = np.maximum(tr["z"] > 0, relu_amb).astype(np.float32)
        E = (np.where(relu_amb, np.abs(tr["da"]), 0.0) + gate * da_chg).astype(np.float32)
        aW, ab = np.zeros_like(Wt), np.zeros(oc, np.float32)
        adx = np.zeros(N * ic * H * W, np.float32)
        oracle.cnref_conv2d_backward(_fp(np.abs(tr["x"])), _fp(np.abs(Wt)), _fp(E), _fp(aW), _fp(ab),
                                     _fp(adx), N, ic, H, W, oc, k, s, p)
        allow[2 * i], allow[2 * i + 1] = aW, ab
        carry = adx
    return allow + [np.zeros(1, np.float32), np.zeros(1, np.float32)]
