"""GPU parity of Conv2D / MaxPool2D (config 3 rows) against the CPU oracle.

Conv: the implicit-GEMM results are contractions, so the relative part of
the rel 1e-4 / abs 1e-5 bound is taken against max(|ref|, mag), mag = the
same contraction of |inputs| divided by sqrt(contraction length)
(oracle_lib.close_mag).  MaxPool: values and int32 argmax bit-exact; dX
bit-exact for non-overlapping windows (one term per element) and within
rel 1e-6 for overlapping ones (a different order of a few additions).
"""
import numpy as np
import pytest
import torch

from oracle import ip
from oracle_lib import close, close_mag, fp

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


CONV_CASES = [(2, 3, 8, 8, 4, 3, 1, 1), (3, 2, 7, 5, 5, 3, 2, 0), (1, 4, 6, 6, 2, 2, 2, 1),
              (4, 3, 5, 5, 3, 1, 1, 0), (5, 5, 9, 7, 40, 5, 1, 2), (8, 70, 6, 6, 33, 3, 1, 1),
              (256, 3, 32, 32, 32, 3, 1, 1), (256, 32, 16, 16, 64, 3, 1, 1),
              # C*KS^2 and OC*KS^2 above the per-block gather-table limit (4608):
              # forward and dgrad take the decoding loaders
              (2, 520, 4, 4, 520, 3, 1, 1),
              # stride 2 with padding, N not a multiple of 4 (scalar wgrad loads)
              (70, 6, 9, 9, 8, 3, 2, 1),
              # N a multiple of the wgrad k-tile (one output pixel per k-tile):
              # 32x64 tile split over 2 wave groups with a partial OC tile, and a
              # 64x32 tile split over 2 wave groups with stride 2
              (32, 6, 8, 8, 20, 3, 1, 1), (16, 3, 10, 10, 48, 3, 2, 1),
              # short contractions (C*KS^2 <= 32, OC % 32 == 0, N % 64 == 0) take the
              # direct MFMA kernel: 5x5 taps with padding 2; stride 2 with no padding on
              # a non-square input and 64 channels; N = 320, whose second sample block
              # has one wave's worth of samples
              (64, 1, 12, 12, 32, 5, 1, 2), (128, 2, 9, 7, 64, 3, 2, 0), (320, 3, 6, 6, 32, 3, 1, 1),
              # OC = 64, C*KS^2 <= 288, N % 32 == 0, N >= 128: the weight gradient takes one
              # output pixel per block (config 3's conv2 above is one): the full 288 columns;
              # 144 columns with stride 2 and no padding on a non-square input; a 1x1 kernel
              (128, 32, 8, 8, 64, 3, 1, 1), (128, 16, 9, 7, 64, 3, 2, 0), (160, 40, 5, 5, 64, 1, 1, 0)]


@pytest.mark.parametrize("N,C,H,W,OC,KS,S,P", CONV_CASES)
@pytest.mark.parametrize("bias", [True, False])
def test_conv2d_vs_oracle(gpu, oracle, N, C, H, W, OC, KS, S, P, bias):
    if bias is False and N == 256:
        pytest.skip("bias-free path covered at the small shapes")
    print(f"[conv2d] N={N} C={C} H={H} W={W} OC={OC} KS={KS} S={S} P={P} bias={bias}", flush=True)
    oracle.cnref_set_threads(16)
    rng = np.random.default_rng(N + C + OC + KS)
    HO, WO = (H + 2 * P - KS) // S + 1, (W + 2 * P - KS) // S + 1
    X = rng.uniform(0, 1, N * C * H * W).astype(np.float32)
    lim = np.sqrt(6.0 / (C * KS * KS + OC * KS * KS))  # conv2d.cpp:42-50 xavier limit
    Wt = rng.uniform(-lim, lim, OC * C * KS * KS).astype(np.float32)
    b = rng.standard_normal(OC).astype(np.float32) if bias else None
    dY = (rng.standard_normal(N * OC * HO * WO) * 1e-3).astype(np.float32)

    Y = torch.empty(N * OC * HO * WO, device="cuda")
    from cppnet_amd import ops
    ops.conv2d_forward(dev(X), dev(Wt), None if b is None else dev(b), Y, N, C, H, W, OC, KS, S, P)
    # the ReLU-fused forward equals the forward then the elementwise ReLU, bit for bit
    Yr, Yr2 = torch.empty_like(Y), torch.empty_like(Y)
    ops.conv2d_forward_relu(dev(X), dev(Wt), None if b is None else dev(b), Yr, N, C, H, W, OC, KS,
                            S, P)
    ops.relu_forward(Y, Yr2)
    np.testing.assert_array_equal(host(Yr), host(Yr2))
    gW = torch.full((OC * C * KS * KS,), 7.0, device="cuda")  # must be overwritten
    gb = torch.full((OC,), 7.0, device="cuda") if bias else None
    dX = torch.empty(N * C * H * W, device="cuda")
    ops.conv2d_backward(dev(X), dev(Wt), dev(dY), gW, gb, dX, N, C, H, W, OC, KS, S, P)

    rY = np.zeros(N * OC * HO * WO, np.float32)
    oracle.cnref_conv2d_forward(fp(X), fp(Wt), fp(b), fp(rY), N, C, H, W, OC, KS, S, P)
    rgW, rgb, rdX = np.zeros_like(Wt), np.zeros(OC, np.float32), np.zeros_like(X)
    oracle.cnref_conv2d_backward(fp(X), fp(Wt), fp(dY), fp(rgW), fp(rgb), fp(rdX), N, C, H, W, OC,
                                 KS, S, P)
    # magnitudes: the same contractions over |inputs|
    mY = np.zeros_like(rY)
    oracle.cnref_conv2d_forward(fp(np.abs(X)), fp(np.abs(Wt)), None, fp(mY), N, C, H, W, OC, KS, S, P)
    mgW, mgb, mdX = np.zeros_like(Wt), np.zeros(OC, np.float32), np.zeros_like(X)
    oracle.cnref_conv2d_backward(fp(np.abs(X)), fp(np.abs(Wt)), fp(np.abs(dY)), fp(mgW), fp(mgb),
                                 fp(mdX), N, C, H, W, OC, KS, S, P)
    for got, want, mag, name in [
            (host(Y), rY, mY / np.sqrt(C * KS * KS), "Y"),
            (host(gW), rgW, mgW / np.sqrt(N * HO * WO), "grad_W"),
            (host(dX), rdX, mdX / np.sqrt(OC * KS * KS), "dX")] + (
            [(host(gb), rgb, mgb / np.sqrt(N * HO * WO), "grad_b")] if bias else []):
        ok, msg = close_mag(got, want, mag, 1e-4, 1e-5)
        assert ok, f"{name}: {msg}"


POOL_CASES = [(2, 3, 8, 8, 2, 2), (3, 2, 5, 5, 3, 1), (1, 4, 7, 9, 2, 3), (4, 2, 6, 6, 3, 2),
              (7, 3, 4, 4, 2, -1), (256, 32, 32, 32, 2, 2), (256, 64, 16, 16, 2, 2),
              (300, 3, 6, 6, 2, 2), (70, 5, 7, 7, 3, 2), (5, 2, 7, 7, 2, 2), (8, 3, 9, 9, 3, 3),
              (12, 2, 7, 7, 2, 2)]


@pytest.mark.parametrize("N,C,H,W,p,s", POOL_CASES)
def test_maxpool_vs_oracle(gpu, oracle, N, C, H, W, p, s):
    print(f"[maxpool] N={N} C={C} H={H} W={W} pool={p} stride={s}", flush=True)
    rng = np.random.default_rng(N + C + H + W + p)
    st = s if s > 0 else p
    HO, WO = (H - p) // st + 1, (W - p) // st + 1
    # quantised values: many exact ties, so "first maximum wins" is exercised
    X = rng.integers(0, 6, N * C * H * W).astype(np.float32)
    X[: min(8, X.size)] = -np.inf
    dY = rng.standard_normal(N * C * HO * WO).astype(np.float32)
    Y = torch.empty(N * C * HO * WO, device="cuda")
    I = torch.empty(N * C * HO * WO, dtype=torch.int32, device="cuda")
    dX = torch.full((N * C * H * W,), 3.0, device="cuda")  # every element must be written
    from cppnet_amd import ops
    ops.maxpool2d_forward(dev(X), Y, I, N, C, H, W, p, s)
    ops.maxpool2d_backward(dev(dY), I, dX, N, C, H, W, p, s)
    rY, rI = np.zeros(N * C * HO * WO, np.float32), np.zeros(N * C * HO * WO, np.int32)
    oracle.cnref_maxpool2d_forward(fp(X), fp(rY), ip(rI), N, C, H, W, p, st)
    rdX = np.zeros_like(X)
    oracle.cnref_maxpool2d_backward(fp(dY), ip(rI), fp(rdX), N, C, H, W, p, st)
    np.testing.assert_array_equal(host(Y), rY)
    np.testing.assert_array_equal(host(I), rI)
    if st >= p:
        np.testing.assert_array_equal(host(dX), rdX)
    else:
        ok, msg = close(host(dX), rdX, 1e-6, 1e-7)
        assert ok, msg
    # every upstream gradient lands somewhere exactly once
    assert abs(float(host(dX).sum()) - float(dY.sum())) <= 1e-3 * max(1.0, float(np.abs(dY).sum()))
    # fused ReLU backward (X stands in for the ReLU output: its zeros and -inf
    # give mask 0): bit-identical to the unfused pair, dX * [y > 0]
    dXr = torch.full((N * C * H * W,), 3.0, device="cuda")
    ops.maxpool2d_backward_relu(dev(dY), I, dev(X), dXr, N, C, H, W, p, s)
    np.testing.assert_array_equal(host(dXr), host(dX) * (X > 0).astype(np.float32))


# Conv2D -> ReLU -> MaxPool2D in one call: the short-contraction fused kernel
# (C*KS^2 <= 32, OC % 32 == 0, N % 64 == 0, pool == stride tiling the conv
# output: config 3's first layer, 2 channel chunks, an unpadded conv, pool 3)
# and the two-step path of every other shape (config 3's second layer, ragged
# batch and channels, a pool that does not tile, overlapping windows)
FUSED_POOL_CASES = [(256, 3, 32, 32, 32, 3, 1, 1, 2, -1), (64, 3, 16, 16, 64, 3, 1, 1, 2, -1),
                    (128, 2, 12, 12, 32, 3, 1, 0, 2, -1), (64, 3, 18, 18, 32, 3, 1, 1, 3, -1),
                    (64, 32, 16, 16, 64, 3, 1, 1, 2, -1), (20, 3, 9, 9, 8, 3, 1, 1, 2, -1),
                    (64, 3, 11, 11, 32, 3, 1, 1, 3, 2)]


@pytest.mark.parametrize("N,C,H,W,OC,KS,S,P,p,ps", FUSED_POOL_CASES)
def test_conv_relu_maxpool_fused(gpu, N, C, H, W, OC, KS, S, P, p, ps):
    """cnhip_conv2d_forward_relu_maxpool against conv + ReLU then max-pool
    (pooled output and argmax bit for bit), and the pool's backward with the
    mask taken from its output against the mask taken from the ReLU output."""
    from cppnet_amd import ops
    print(f"[conv-relu-pool] N={N} C={C} H={H} W={W} OC={OC} KS={KS} S={S} P={P} pool={p} stride={ps}", flush=True)
    rng = np.random.default_rng(N + C + H + OC + p)
    X = rng.standard_normal(N * C * H * W).astype(np.float32)
    # quantised weights: exact ties and exact zeros after the ReLU
    Wt = (rng.integers(-3, 4, OC * C * KS * KS) * 0.25).astype(np.float32)
    b = (rng.integers(-2, 3, OC) * 0.5).astype(np.float32)
    HO, WO = (H + 2 * P - KS) // S + 1, (W + 2 * P - KS) // S + 1
    st = ps if ps > 0 else p
    HP, WP = (HO - p) // st + 1, (WO - p) // st + 1
    Y1 = torch.empty(N * OC * HO * WO, device="cuda")
    ops.conv2d_forward_relu(dev(X), dev(Wt), dev(b), Y1, N, C, H, W, OC, KS, S, P)
    Yp, I = torch.empty(N * OC * HP * WP, device="cuda"), torch.empty(N * OC * HP * WP, dtype=torch.int32, device="cuda")
    ops.maxpool2d_forward(Y1, Yp, I, N, OC, HO, WO, p, ps)
    Fp = torch.full((N * OC * HP * WP,), 7.0, device="cuda")
    FI = torch.full((N * OC * HP * WP,), -1, dtype=torch.int32, device="cuda")
    ops.conv2d_forward_relu_maxpool(dev(X), dev(Wt), dev(b), Fp, FI, N, C, H, W, OC, KS, S, P, p, ps)
    assert np.array_equal(host(Fp).view(np.uint32), host(Yp).view(np.uint32))
    assert np.array_equal(host(FI), host(I))
    dYp = rng.standard_normal(N * OC * HP * WP).astype(np.float32)
    dA = torch.full((N * OC * HO * WO,), 3.0, device="cuda")
    dB = torch.full((N * OC * HO * WO,), 5.0, device="cuda")
    ops.maxpool2d_backward_relu(dev(dYp), I, Y1, dA, N, OC, HO, WO, p, ps)
    ops.maxpool2d_backward_relu_pooled(dev(dYp), FI, Fp, dB, N, OC, HO, WO, p, ps)
    if st == p and HP * p == HO and WP * p == WO:
        assert np.array_equal(host(dB).view(np.uint32), host(dA).view(np.uint32))
    else:
        np.testing.assert_array_equal(host(dB), host(dA))


# (N, C, H, W, OC, KS, S, P, pool): config 3's first layer; more channels and
# the 64 x 64 weight-gradient tile (OC 64, 289 columns); an unpadded conv with
# pool 3; stride 2 with padding 2; no bias
CONV_POOL_BWD_CASES = [(256, 3, 32, 32, 32, 3, 1, 1, 2, True), (64, 32, 16, 16, 64, 3, 1, 1, 2, True),
                       (128, 2, 14, 14, 32, 3, 1, 0, 3, True), (64, 4, 19, 19, 16, 5, 2, 2, 2, True),
                       (64, 3, 16, 16, 32, 3, 1, 1, 2, False)]


@pytest.mark.parametrize("N,C,H,W,OC,KS,S,P,p,bias", CONV_POOL_BWD_CASES)
def test_conv_backward_maxpool_relu_fused(gpu, N, C, H, W, OC, KS, S, P, p, bias):
    """cnhip_conv2d_backward_maxpool_relu (the conv's weight and bias
    gradients formed from the pooled gradient, argmax and pooled output)
    against cnhip_maxpool2d_backward_relu_pooled then cnhip_conv2d_backward:
    bit for bit, on quantised weights with exact ties and exact zeros."""
    from cppnet_amd import ops
    print(f"[conv-pool-bwd] N={N} C={C} H={H} W={W} OC={OC} KS={KS} S={S} P={P} pool={p} bias={bias}", flush=True)
    rng = np.random.default_rng(N + 3 * C + H + OC + p + KS)
    X = rng.standard_normal(N * C * H * W).astype(np.float32)
    Wt = (rng.integers(-3, 4, OC * C * KS * KS) * 0.25).astype(np.float32)
    b = (rng.integers(-2, 3, OC) * 0.5).astype(np.float32)
    HO, WO = (H + 2 * P - KS) // S + 1, (W + 2 * P - KS) // S + 1
    HP, WP = HO // p, WO // p
    assert ops.conv2d_backward_maxpool_relu_fits(N, C, H, W, OC, KS, S, P, p)
    Fp = torch.empty(N * OC * HP * WP, device="cuda")
    FI = torch.empty(N * OC * HP * WP, dtype=torch.int32, device="cuda")
    ops.conv2d_forward_relu_maxpool(dev(X), dev(Wt), dev(b), Fp, FI, N, C, H, W, OC, KS, S, P, p)
    dP = dev(rng.standard_normal(N * OC * HP * WP).astype(np.float32))
    dZ = torch.empty(N * OC * HO * WO, device="cuda")
    ops.maxpool2d_backward_relu_pooled(dP, FI, Fp, dZ, N, OC, HO, WO, p)
    gW0, gb0 = torch.full((OC * C * KS * KS,), 7.0, device="cuda"), torch.full((OC,), 7.0, device="cuda")
    ops.conv2d_backward(dev(X), dev(Wt), dZ, gW0, gb0 if bias else None, None, N, C, H, W, OC, KS, S, P)
    gW1, gb1 = torch.full((OC * C * KS * KS,), 9.0, device="cuda"), torch.full((OC,), 9.0, device="cuda")
    ops.conv2d_backward_maxpool_relu(dev(X), dP, FI, Fp, gW1, gb1 if bias else None, N, C, H, W, OC, KS, S, P, p)
    assert np.array_equal(host(gW1).view(np.uint32), host(gW0).view(np.uint32))
    if bias:
        assert np.array_equal(host(gb1).view(np.uint32), host(gb0).view(np.uint32))
    else:
        assert bool((gb1 == 9.0).all())


def test_conv_backward_maxpool_relu_refuses_unfit_shapes(gpu):
    """Shapes the fused weight gradient does not take are reported by _fits
    and refused by the call (a batch that is no multiple of 64; windows that
    do not tile the conv output; overlapping windows) before any work."""
    from cppnet_amd import _capi, ops
    assert not ops.conv2d_backward_maxpool_relu_fits(100, 3, 16, 16, 32, 3, 1, 1, 2)
    assert not ops.conv2d_backward_maxpool_relu_fits(64, 3, 15, 15, 32, 3, 1, 1, 2)
    assert not ops.conv2d_backward_maxpool_relu_fits(64, 3, 16, 16, 32, 3, 1, 1, 3, 2)
    N, C, H, W, OC = 100, 3, 16, 16, 32
    t = torch.zeros(N * OC * 8 * 8, device="cuda")
    ti = torch.zeros(N * OC * 8 * 8, dtype=torch.int32, device="cuda")
    gW = torch.full((OC * C * 9,), 7.0, device="cuda")
    with pytest.raises(_capi.CnhipError, match="N % 64"):
        ops.conv2d_backward_maxpool_relu(torch.zeros(N * C * H * W, device="cuda"), t, ti, t, gW, None,
                                         N, C, H, W, OC, 3, 1, 1, 2)
    assert bool((gW == 7.0).all())


# (N, C, H, W, O, pool): config 3's head; a batch that is no multiple of 64;
# a batch of at most 64 (the separate weight gradient then sums on one thread,
# so only the tolerance applies) with 3x3 windows and 16 outputs; the largest
# staged dZ (N O = 8192); more outputs than pooled features
HEAD_POOL_CASES = [(256, 64, 16, 16, 10, 2), (100, 3, 6, 4, 3, 2), (32, 5, 6, 6, 16, 3), (512, 8, 4, 4, 16, 2),
                   # fewer features (2) than outputs (13): the bias columns take waves of their own
                   (96, 2, 2, 2, 13, 2),
                   # a batch above 64 and no multiple of 4: the lane-strided kernel
                   (130, 3, 4, 4, 5, 2)]


@pytest.mark.parametrize("N,C,H,W,O,p", HEAD_POOL_CASES)
@pytest.mark.parametrize("accumulate", [0, 1])
def test_linear_backward_maxpool_relu(gpu, N, C, H, W, O, p, accumulate):
    """cnhip_linear_backward_maxpool_relu (Linear + Flatten + MaxPool2D + ReLU
    backward in one pass) against a float64 restatement (close_mag bound) and
    against the separate calls cnhip_linear_backward then
    cnhip_maxpool2d_backward_relu_pooled: dX routed to the same elements with
    values within the contraction bound (the separate dX is an MFMA product,
    summed in another order), and, for a batch that is no multiple of 4 (the
    lane-strided kernel) above 64, grad_W and grad_b bit for bit those of the
    separate wave-per-output weight-gradient kernel."""
    from cppnet_amd import ops
    print(f"[linear-pool-bwd] N={N} C={C} H={H} W={W} O={O} pool={p} acc={accumulate}", flush=True)
    rng = np.random.default_rng(N + C + H + W + O + p + accumulate)
    HO, WO = H // p, W // p
    F = C * HO * WO
    # a ReLU output with exact zeros and ties, pooled on the GPU
    Y = np.maximum(rng.integers(-4, 5, N * C * H * W) * 0.5, 0).astype(np.float32)
    Pt = torch.empty(N * F, device="cuda")
    It = torch.empty(N * F, dtype=torch.int32, device="cuda")
    ops.maxpool2d_forward(dev(Y), Pt, It, N, C, H, W, p, -1)
    Wt = rng.standard_normal(F * O).astype(np.float32)
    dZ = rng.standard_normal(N * O).astype(np.float32)
    gW0 = rng.standard_normal(F * O).astype(np.float32)
    gb0 = rng.standard_normal(O).astype(np.float32)
    assert ops.linear_backward_maxpool_relu_fits(N, C, H, W, O, p, -1)
    gWa, gba = dev(gW0), dev(gb0)
    dXa = torch.full((N * C * H * W,), 9.0, device="cuda")
    ops.linear_backward_maxpool_relu(Pt, It, dev(Wt), dev(dZ), gWa, gba, dXa, N, C, H, W, O, p, -1, accumulate)
    gWb, gbb = dev(gW0), dev(gb0)
    dP = torch.empty(N * F, device="cuda")
    dXb = torch.full((N * C * H * W,), 7.0, device="cuda")
    ops.linear_backward(Pt, dev(Wt), dev(dZ), gWb, gbb, dP, N, F, O, True, bool(accumulate))
    ops.maxpool2d_backward_relu_pooled(dP, It, Pt, dXb, N, C, H, W, p, -1)
    P, I = host(Pt), host(It)
    # float64 restatement
    Pm, dZm, Wm = P.reshape(F, N).T.astype(np.float64), dZ.reshape(O, N).T.astype(np.float64), \
        Wt.reshape(O, F).T.astype(np.float64)
    gW_ref = (Pm.T @ dZm).T.reshape(-1) + (gW0 if accumulate else 0)
    gW_mag = (np.abs(Pm).T @ np.abs(dZm)).T.reshape(-1) / np.sqrt(N)
    gb_ref = dZm.sum(0) + (gb0 if accumulate else 0)
    g = (dZm @ Wm.T).T.reshape(WO, HO, C, N) * (P.reshape(WO, HO, C, N) > 0)
    gmag = (np.abs(dZm) @ np.abs(Wm).T).T.reshape(WO, HO, C, N) / np.sqrt(O)
    I4 = I.reshape(WO, HO, C, N)
    dX_ref = np.zeros((WO, p, HO, p, C, N))
    dX_mag = np.zeros((WO, p, HO, p, C, N))
    for ph in range(p):
        for pw in range(p):
            hit = I4 == ph * p + pw
            dX_ref[:, pw, :, ph] = np.where(hit, g, 0.0)
            dX_mag[:, pw, :, ph] = np.where(hit, gmag, 0.0)
    dXa_h, dXb_h = host(dXa), host(dXb)
    for name, a, ref, mag in (("grad_W", host(gWa), gW_ref, gW_mag), ("dX", dXa_h, dX_ref.reshape(-1), dX_mag.reshape(-1))):
        ok, msg = close_mag(a, ref, mag)
        assert ok, f"{name}: {msg}"
    ok, msg = close_mag(host(gba), gb_ref, np.abs(dZm).sum(0) / np.sqrt(N))
    assert ok, f"grad_b: {msg}"
    # the separate calls: the same routing (every element written, zeros where
    # the pool routes nothing), values within the bound
    assert np.array_equal(dXa_h == 0, dXb_h == 0)
    ok, msg = close_mag(dXa_h, dXb_h, dX_mag.reshape(-1))
    assert ok, f"dX vs separate calls: {msg}"
    if N > 64 and N % 4 != 0:
        assert np.array_equal(host(gWa).view(np.uint32), host(gWb).view(np.uint32))
        assert np.array_equal(host(gba).view(np.uint32), host(gbb).view(np.uint32))
