"""GPU parity of the C-ABI ops against the CPU oracle (same seeded inputs).

Tolerances: fp32 results within rel 1e-4 / abs 1e-5 of the oracle,
elementwise |gpu - ref| <= 1e-5 + 1e-4*|ref|; for contractions (GEMM,
Linear, column sums) the relative part is taken against
max(|ref|, (|A||B|)/sqrt(K)), the RMS size of the dot product's partial
sums, since a cancelled fp32 sum carries ~u*sqrt(K) of that size on both
sides (oracle_lib.close_mag).  Adam is checked
bit-exact: the kernel evaluates the reference's operation sequence without
contraction, and fp32 division/sqrt are correctly rounded on both sides.
"""
import numpy as np
import pytest
import torch

from cppnet_amd import ops
from oracle_lib import close, close_mag, fp, gemm_mag

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-4, 1e-5


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def rnd(rng, n, scale=1.0):
    return (rng.standard_normal(n) * scale).astype(np.float32)


def _gemm_case(oracle, ta, tb, M, N, K, beta, with_bias, relu, pad, seed):
    rng = np.random.default_rng(seed)
    lda = (K if ta else M) + pad
    ldb = (N if tb else K) + pad
    ldc = M + pad
    A = rnd(rng, max(1, lda * (M if ta else K)))
    B = rnd(rng, max(1, ldb * (K if tb else N)))
    C = rnd(rng, ldc * N)
    bias = rnd(rng, N) if with_bias else None
    Cd = dev(C)
    ops.gemm(ta, tb, M, N, K, dev(A), lda, dev(B), ldb, Cd, ldc, alpha=1.0, beta=beta,
             bias=None if bias is None else dev(bias), relu=relu)
    want = C.copy()
    oracle.cnref_gemm_f32(ta, tb, M, N, K, 1.0, fp(A), lda, fp(B), ldb, beta, fp(want), ldc,
                          fp(bias), 1 if relu else 0)
    got = host(Cd)
    mag = gemm_mag(oracle, ta, tb, M, N, K, A, lda, B, ldb, ldc)
    ok, msg = close_mag(got, want, mag, RTOL, ATOL)
    assert ok, f"gemm ta={ta} tb={tb} M={M} N={N} K={K}: {msg}"


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(128, 128, 16), (256, 384, 512), (130, 70, 33), (1, 1, 1),
                                   (5, 300, 7), (300, 10, 700), (64, 3, 2000), (512, 512, 10),
                                   (1024, 512, 2048), (512, 1024, 2048), (1000, 520, 2050)])
def test_gemm_vs_oracle(gpu, oracle, ta, tb, M, N, K):
    print(f"[gemm] ta={ta} tb={tb} M={M} N={N} K={K}", flush=True)
    _gemm_case(oracle, ta, tb, M, N, K, beta=0.0, with_bias=False, relu=False, pad=0, seed=M + N + K)


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1)])
def test_gemm_epilogues_and_strides(gpu, oracle, ta, tb):
    print(f"[gemm-epi] ta={ta} tb={tb}", flush=True)
    _gemm_case(oracle, ta, tb, 200, 150, 96, beta=1.0, with_bias=True, relu=True, pad=3, seed=11)
    _gemm_case(oracle, ta, tb, 129, 257, 300, beta=0.5, with_bias=True, relu=False, pad=1, seed=12)


def test_gemm_k_zero_scales_c(gpu, oracle):
    _gemm_case(oracle, 0, 0, 40, 30, 0, beta=1.0, with_bias=True, relu=False, pad=0, seed=3)


# (4096, 1024, 10) .. (8192, 512, 1) take the one-pass backward of a few-output
# layer (O in 1, 2, 4, 8, 10, 16; B % 512 == 0, I % 16 == 0, B*I >= 2^22) and
# the one-pass forward (B % 256 == 0, I % 64 == 0, B*I >= 2^20), as does
# config 3's head (256, 4096, 10) for the forward only; (4100, 1100, 3) is
# just outside both; (8192, 512, 2048) runs dX and dW in one launch (both on
# 128 x 128 tiles, 256 blocks each)
@pytest.mark.parametrize("B,I,O", [(512, 30, 64), (512, 64, 1), (256, 1024, 256), (33, 17, 5),
                                   (4096, 1024, 10), (2048, 2048, 16), (1024, 4096, 8), (4096, 1024, 4),
                                   (8192, 512, 2), (8192, 512, 1), (256, 4096, 10), (4100, 1100, 3),
                                   (8192, 512, 2048)])
@pytest.mark.parametrize("trainable", [1, 0])
def test_linear_vs_oracle(gpu, oracle, B, I, O, trainable):
    print(f"[linear] B={B} I={I} O={O} trainable={trainable}", flush=True)
    rng = np.random.default_rng(B * 7 + I + O)
    X, W, b = rnd(rng, B * I), rnd(rng, I * O, 0.1), rnd(rng, O)
    dY = rnd(rng, B * O, 0.01)
    gW0, gb0 = rnd(rng, I * O, 1e-3), rnd(rng, O, 1e-3)
    Y = torch.empty(B * O, device="cuda")
    ops.linear_forward(dev(X), dev(W), dev(b), Y, B, I, O)
    gW, gb, dX = dev(gW0), dev(gb0), torch.empty(B * I, device="cuda")
    ops.linear_backward(dev(X), dev(W), dev(dY), gW, gb, dX, B, I, O, trainable=bool(trainable),
                        accumulate=True)
    rY = np.zeros(B * O, np.float32)
    oracle.cnref_linear_forward(fp(X), fp(W), fp(b), fp(rY), B, I, O)
    rgW, rgb, rdX = gW0.copy(), gb0.copy(), np.zeros(B * I, np.float32)
    oracle.cnref_linear_backward(fp(X), fp(W), fp(dY), fp(rgW), fp(rgb), fp(rdX), B, I, O,
                                 trainable, 1)
    mags = {"Y": gemm_mag(oracle, 0, 0, B, O, I, X, B, W, I, B),
            "grad_W": gemm_mag(oracle, 1, 0, I, O, B, X, B, dY, B, I),
            "grad_b": gemm_mag(oracle, 1, 0, 1, O, B, np.ones(B, np.float32), B, dY, B, 1),
            "dX": gemm_mag(oracle, 0, 1, B, I, O, dY, B, W, I, B)}
    for got, want, name in [(host(Y), rY, "Y"), (host(gW), rgW, "grad_W"),
                            (host(gb), rgb, "grad_b"), (host(dX), rdX, "dX")]:
        ok, msg = close_mag(got, want, mags[name], RTOL, ATOL)
        assert ok, f"{name}: {msg}"


def test_linear_accumulates_over_two_backwards(gpu, oracle):
    B, I, O = 64, 40, 24
    rng = np.random.default_rng(2)
    X, W, dY = rnd(rng, B * I), rnd(rng, I * O), rnd(rng, B * O)
    gW, gb = torch.zeros(I * O, device="cuda"), torch.zeros(O, device="cuda")
    for _ in range(2):
        ops.linear_backward(dev(X), dev(W), dev(dY), gW, gb, None, B, I, O)
    rgW, rgb = np.zeros(I * O, np.float32), np.zeros(O, np.float32)
    for _ in range(2):
        oracle.cnref_linear_backward(fp(X), fp(W), fp(dY), fp(rgW), fp(rgb), None, B, I, O, 1, 1)
    mag = 2 * gemm_mag(oracle, 1, 0, I, O, B, X, B, dY, B, I)
    assert close_mag(host(gW), rgW, mag, RTOL, ATOL)[0]
    assert close_mag(host(gb), rgb, 2 * gemm_mag(oracle, 1, 0, 1, O, B, np.ones(B, np.float32), B,
                                                  dY, B, 1), RTOL, ATOL)[0]


@pytest.mark.parametrize("rows,cols", [(4096, 37), (7, 3), (1, 5), (1000, 1)])
def test_column_sum(gpu, oracle, rows, cols):
    rng = np.random.default_rng(rows + cols)
    a = rnd(rng, rows * cols)
    out0 = rnd(rng, cols)
    out = dev(out0)
    ops.column_sum(dev(a), out, rows, cols, accumulate=True)
    want = out0.copy()
    oracle.cnref_column_sum(fp(a), fp(want), rows, cols, 1)
    mag = gemm_mag(oracle, 1, 0, 1, cols, rows, np.ones(rows, np.float32), rows, a, rows, 1)
    ok, msg = close_mag(host(out), want, mag, RTOL, ATOL)
    assert ok, msg


@pytest.mark.parametrize("name", ["relu", "sigmoid", "tanh"])
@pytest.mark.parametrize("n", [1, 3, 4, 1001, 4096 * 64])
def test_activation_vs_oracle(gpu, oracle, name, n):
    rng = np.random.default_rng(n)
    x = rnd(rng, n, 4.0)
    if n > 3:
        x[:3] = [0.0, 700.0, -700.0]
    dy = rnd(rng, n)
    y, dx = torch.empty(n, device="cuda"), torch.empty(n, device="cuda")
    getattr(ops, f"{name}_forward")(dev(x), y)
    getattr(ops, f"{name}_backward")(y, dev(dy), dx)
    ry, rdx = np.zeros(n, np.float32), np.zeros(n, np.float32)
    getattr(oracle, f"cnref_{name}_forward")(fp(x), fp(ry), n)
    # the backward is checked on the GPU's own forward output, so a 1-ulp
    # difference in exp/tanh does not leak into the derivative check
    y_h = host(y)
    getattr(oracle, f"cnref_{name}_backward")(fp(y_h), fp(dy), fp(rdx), n)
    ok, msg = close(y_h, ry, RTOL, ATOL)
    assert ok, f"{name} forward: {msg}"
    got_dx = host(dx)
    if name == "relu":
        np.testing.assert_array_equal(got_dx, rdx)
        np.testing.assert_array_equal(y_h, ry)
    ok, msg = close(got_dx, rdx, RTOL, ATOL)
    assert ok, f"{name} backward: {msg}"


@pytest.mark.parametrize("n", [1, 512, 10000])
@pytest.mark.parametrize("reduction", ["mean", "sum"])
def test_bce_vs_oracle(gpu, oracle, n, reduction):
    rng = np.random.default_rng(n)
    p = rng.uniform(0.0, 1.0, n).astype(np.float32)
    p[: min(n, 2)] = [0.0, 1.0][: min(n, 2)]
    t = (rng.uniform(size=n) < 0.5).astype(np.float32)
    loss, g = torch.empty(1, device="cuda"), torch.empty(n, device="cuda")
    ops.bce_forward(dev(p), dev(t), loss, reduction)
    ops.bce_backward(dev(p), dev(t), g, reduction)
    r = 0 if reduction == "mean" else 1
    want = oracle.cnref_bce_forward(fp(p), fp(t), n, r)
    rg = np.zeros(n, np.float32)
    oracle.cnref_bce_backward(fp(p), fp(t), fp(rg), n, r)
    ok, msg = close(host(loss), [want], RTOL, ATOL)
    assert ok, msg
    ok, msg = close(host(g), rg, RTOL, ATOL)
    assert ok, msg


@pytest.mark.parametrize("n", [1, 128, 9999, 65536])
@pytest.mark.parametrize("reduction", ["mean", "sum"])
def test_mse_vs_oracle(gpu, oracle, n, reduction):
    rng = np.random.default_rng(n + 1)
    p, t = rnd(rng, n), rnd(rng, n)
    loss, g = torch.empty(1, device="cuda"), torch.empty(n, device="cuda")
    ops.mse_forward(dev(p), dev(t), loss, reduction)
    ops.mse_backward(dev(p), dev(t), g, reduction)
    r = 0 if reduction == "mean" else 1
    rg = np.zeros(n, np.float32)
    oracle.cnref_mse_backward(fp(p), fp(t), fp(rg), n, r)
    ok, msg = close(host(loss), [oracle.cnref_mse_forward(fp(p), fp(t), n, r)], RTOL, ATOL)
    assert ok, msg
    np.testing.assert_array_equal(host(g), rg)
    # the one-launch form: the same loss and gradient bits
    loss2, g2 = torch.empty(1, device="cuda"), torch.empty(n, device="cuda")
    ops.mse_head(dev(p), dev(t), loss2, g2, reduction)
    assert torch.equal(loss2, loss) and torch.equal(g2, g)


@pytest.mark.parametrize("B,Cc", [(1, 3), (4096, 10), (256, 10), (32, 4), (77, 1)])
def test_softmax_ce_vs_oracle(gpu, oracle, B, Cc):
    rng = np.random.default_rng(B + Cc)
    z = rnd(rng, B * Cc, 3.0)
    labels = rng.integers(0, Cc, B)
    t = np.zeros((Cc, B), np.float32)
    t[labels, np.arange(B)] = 1.0  # ColMajor [B, C]: column c holds class c
    t = t.ravel()
    sm, loss = torch.empty(B * Cc, device="cuda"), torch.empty(1, device="cuda")
    g = torch.empty(B * Cc, device="cuda")
    ops.softmax_ce_forward(dev(z), dev(t), sm, loss, B, Cc)
    ops.softmax_ce_backward(sm, dev(t), g, B, Cc)
    rsm, rg = np.zeros(B * Cc, np.float32), np.zeros(B * Cc, np.float32)
    want = oracle.cnref_softmax_ce_forward(fp(z), fp(t), fp(rsm), B, Cc, 0)
    oracle.cnref_softmax_ce_backward(fp(rsm), fp(t), fp(rg), B, Cc, 0)
    for got, ref, name in [(host(loss), [want], "loss"), (host(sm), rsm, "softmax"),
                           (host(g), rg, "grad")]:
        ok, msg = close(got, ref, RTOL, ATOL)
        assert ok, f"{name}: {msg}"


@pytest.mark.parametrize("n", [1, 7, 4096, 4096 * 4096 + 3])
def test_adam_bit_exact(gpu, oracle, n):
    print(f"[adam] n={n}", flush=True)
    rng = np.random.default_rng(n % 1000)
    W, m, v = rnd(rng, n), np.zeros(n, np.float32), np.zeros(n, np.float32)
    Wd, md, vd = dev(W), dev(m), dev(v)
    lr, b1, b2, eps = 1e-3, 0.9, 0.999, 1e-8
    for t in (1, 2, 3):
        g = rnd(rng, n, 0.1)
        bc1, bc2 = oracle.cnref_bias_correction(b1, t), oracle.cnref_bias_correction(b2, t)
        ops.adam_step(Wd, dev(g), md, vd, lr, b1, b2, eps, bc1, bc2)
        oracle.cnref_adam_step(fp(W), fp(g), fp(m), fp(v), n, lr, b1, b2, eps, bc1, bc2)
    np.testing.assert_array_equal(host(Wd), W)
    np.testing.assert_array_equal(host(md), m)
    np.testing.assert_array_equal(host(vd), v)


def test_adam_multi_matches_single(gpu, oracle):
    rng = np.random.default_rng(4)
    sizes = [1024 * 4096, 4096, 10, 3, 4096 * 10]
    lr, b1, b2, eps = 1e-3, 0.9, 0.999, 1e-8
    params, refs = [], []
    for i, n in enumerate(sizes):
        W, g = rnd(rng, n), rnd(rng, n, 0.1)
        t = 1 + i  # distinct per-tensor step counts (per-key t of the reference)
        bc1, bc2 = oracle.cnref_bias_correction(b1, t), oracle.cnref_bias_correction(b2, t)
        m, v = rnd(rng, n, 0.01), np.abs(rnd(rng, n, 0.01))
        params.append((dev(W), dev(g), dev(m), dev(v), bc1, bc2))
        oracle.cnref_adam_step(fp(W), fp(g), fp(m), fp(v), n, lr, b1, b2, eps, bc1, bc2)
        refs.append((W, m, v))
    ops.adam_step_multi(params, lr, b1, b2, eps)
    for (Wd, _, md, vd, _, _), (W, m, v) in zip(params, refs):
        np.testing.assert_array_equal(host(Wd), W)
        np.testing.assert_array_equal(host(md), m)
        np.testing.assert_array_equal(host(vd), v)


def test_gemm_config2_shapes_vs_torch(gpu):
    """Full config-2 GEMM shapes against torch's fp32 matmul (hipBLASLt) as an
    independent float reference (the oracle is too slow at 4096^3 to run per test)."""
    torch.backends.cuda.matmul.allow_tf32 = False
    g = torch.Generator(device="cuda").manual_seed(0)
    for (ta, tb, M, N, K) in [(0, 0, 4096, 4096, 4096), (1, 0, 1024, 4096, 4096),
                              (0, 1, 4096, 1024, 4096), (1, 0, 4096, 10, 4096),
                              (0, 1, 4096, 4096, 10)]:
        print(f"[gemm-c2] ta={ta} tb={tb} M={M} N={N} K={K}", flush=True)
        A = torch.randn((M, K) if ta else (K, M), device="cuda", generator=g)  # row-major storage
        B = torch.randn((N, K) if not tb else (K, N), device="cuda", generator=g)
        # ColMajor views: A_cm(m,k) -> ta ? A[m][k] : A[k][m] etc.
        opA = A if ta else A.t()
        opB = B.t() if not tb else B
        C = torch.empty(N, M, device="cuda")  # ColMajor [M,N] == row-major [N,M]
        ops.gemm(ta, tb, M, N, K, A, K if ta else M, B, K if not tb else N, C, M)
        ref = (opA.double() @ opB.double()).t()
        err = (C.double() - ref).abs()
        lim = 1e-5 + 1e-4 * ref.abs()
        # fp32 sums of K=4096 N(0,1) products: compare elementwise against the
        # fp64 product with the rel/abs bound scaled by sqrt(K) * |row|*|col|
        scale = (opA.double().norm(dim=1)[:, None] * opB.double().norm(dim=0)[None, :]).t()
        bound = torch.maximum(lim, 4e-7 * scale)
        assert bool((err <= bound).all()), f"max err {err.max().item()} at ta={ta} tb={tb} {M}x{N}x{K}"


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1)])
@pytest.mark.parametrize("M,N,K,batch", [(64, 96, 40, 5), (256, 256, 64, 3), (17, 33, 300, 4)])
def test_gemm_batched_vs_oracle(gpu, oracle, ta, tb, M, N, K, batch):
    print(f"[gemm-batched] ta={ta} tb={tb} M={M} N={N} K={K} batch={batch}", flush=True)
    rng = np.random.default_rng(M + N + K + batch)
    lda, ldb, ldc = (K if ta else M) + 1, (N if tb else K) + 2, M + 3
    sa, sb, sc = lda * (M if ta else K) + 5, ldb * (K if tb else N) + 7, ldc * N + 1
    A, B = rnd(rng, sa * batch), rnd(rng, sb * batch)
    C = rnd(rng, sc * batch)
    Cd = dev(C)
    ops.gemm_batched(ta, tb, M, N, K, dev(A), lda, sa, dev(B), ldb, sb, Cd, ldc, sc, batch,
                     alpha=0.5, beta=1.0)
    got = host(Cd)
    for b in range(batch):
        want = C[b * sc:(b + 1) * sc].copy()
        Ab, Bb = A[b * sa:(b + 1) * sa], B[b * sb:(b + 1) * sb]
        oracle.cnref_gemm_f32(ta, tb, M, N, K, 0.5, fp(Ab), lda, fp(Bb), ldb, 1.0, fp(want), ldc,
                              None, 0)
        mag = gemm_mag(oracle, ta, tb, M, N, K, Ab, lda, Bb, ldb, ldc)
        ok, msg = close_mag(got[b * sc:b * sc + ldc * N], want[:ldc * N], mag, RTOL, ATOL)
        assert ok, f"batch {b}: {msg}"
        # padding between batch entries untouched
        np.testing.assert_array_equal(got[b * sc + ldc * N:(b + 1) * sc], C[b * sc + ldc * N:(b + 1) * sc])


@pytest.mark.parametrize("act", ["relu", "gelu"])
# (8192, 2048, 512): the backward's dX and dW run in one launch on both paths
@pytest.mark.parametrize("B,I,O", [(64, 48, 40), (4096, 1024, 512), (37, 130, 19), (4096, 10, 4096),
                                   (8192, 2048, 512)])
def test_linear_fused_activation_matches_unfused(gpu, oracle, act, B, I, O):
    """Linear + activation in one GEMM epilogue, and the next layer's input
    gradient with the activation derivative in its epilogue, equal the
    separate Linear and activation calls bit for bit (same per-element
    arithmetic, same GEMM plan), and the oracle within the contraction bar."""
    print(f"[linear-act] {act} B={B} I={I} O={O}", flush=True)
    rng = np.random.default_rng(B + I + O)
    X, W, b = rnd(rng, B * I), rnd(rng, I * O, 1 / np.sqrt(I)), rnd(rng, O, 0.1)
    dY = rnd(rng, B * O)
    Y, Z = torch.empty(B * O, device="cuda"), torch.empty(B * O, device="cuda")
    ops.linear_forward_act(dev(X), dev(W), dev(b), Y, Z, B, I, O, act)
    Zu, Yu = torch.empty(B * O, device="cuda"), torch.empty(B * O, device="cuda")
    ops.linear_forward(dev(X), dev(W), dev(b), Zu, B, I, O)
    (ops.relu_forward if act == "relu" else ops.gelu_forward)(Zu, Yu)
    np.testing.assert_array_equal(host(Y), host(Yu))
    if act == "gelu":
        np.testing.assert_array_equal(host(Z), host(Zu))
    # backward of a Linear (I2 -> O) stacked on this activation: its dX carries act'
    aux = Yu if act == "relu" else Zu
    W2 = rnd(rng, O * I, 1 / np.sqrt(O))
    gW, gb, dX = torch.empty(O * I, device="cuda"), torch.empty(I, device="cuda"), torch.empty(B * O, device="cuda")
    dY2 = dev(rnd(rng, B * I))
    ops.linear_backward_act(Yu, dev(W2), dY2, gW, gb, dX, aux, B, O, I, act)
    gWu, gbu, dXu = torch.empty(O * I, device="cuda"), torch.empty(I, device="cuda"), torch.empty(B * O, device="cuda")
    ops.linear_backward(Yu, dev(W2), dY2, gWu, gbu, dXu, B, O, I, True, False)
    dZ = torch.empty(B * O, device="cuda")
    if act == "relu":
        ops.relu_backward(aux, dXu, dZ)
    else:
        ops.gelu_backward(aux, dXu, dZ)
    np.testing.assert_array_equal(host(dX), host(dZ))
    np.testing.assert_array_equal(host(gW), host(gWu))
    np.testing.assert_array_equal(host(gb), host(gbu))
    # forward against the oracle (Linear then the activation)
    rz = np.zeros(B * O, np.float32)
    oracle.cnref_linear_forward(fp(X), fp(W), fp(b), fp(rz), B, I, O)
    ry = np.zeros_like(rz)
    (oracle.cnref_relu_forward if act == "relu" else oracle.cnref_gelu_forward)(fp(rz), fp(ry), rz.size)
    mag = gemm_mag(oracle, 0, 0, B, O, I, X, B, W, I, B)
    ok, msg = close_mag(host(Y), ry, mag, 1e-4, 1e-5)
    assert ok, msg


# (128, 512, 1): config 4's head; the rest cover the thread and wave kernels on each side
@pytest.mark.parametrize("B,I,O", [(128, 512, 1), (32, 512, 10), (200, 96, 3), (64, 48, 100), (100, 64, 80)])
@pytest.mark.parametrize("accumulate", [False, True])
def test_linear_backward_small_pair_matches_separate_launches(gpu, B, I, O, accumulate):
    """A small Linear's dW (with db) and dX in one launch equal the layer's
    weight-gradient launch (its backward without dX) followed by a separate
    dX GEMM, bit for bit."""
    print(f"[linear-small-pair] acc={accumulate} B={B} I={I} O={O}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(B * 7 + I + O)
    X = torch.randn(B * I, device="cuda", generator=g)
    W = torch.randn(I * O, device="cuda", generator=g) / np.sqrt(I)
    dY = torch.randn(B * O, device="cuda", generator=g)
    gW0 = torch.randn(I * O, device="cuda", generator=g) * 1e-3
    gb0 = torch.randn(O, device="cuda", generator=g) * 1e-3
    gW, gb, dX = gW0.clone(), gb0.clone(), torch.empty(B * I, device="cuda")
    ops.linear_backward(X, W, dY, gW, gb, dX, B, I, O, True, accumulate)
    gWs, gbs, dXs = gW0.clone(), gb0.clone(), torch.empty(B * I, device="cuda")
    ops.linear_backward(X, W, dY, gWs, gbs, None, B, I, O, True, accumulate)
    ops.gemm(False, True, B, I, O, dY, B, W, I, dXs, B)
    torch.cuda.synchronize()
    assert torch.equal(dX, dXs), "dX"
    assert torch.equal(gW, gWs), "grad_W"
    assert torch.equal(gb, gbs), "grad_b"


@pytest.mark.parametrize("act,accumulate", [("none", False), ("none", True), ("relu", False)])
# (4096, 4096, 4096): config 2's hidden layer, 256 + 256 blocks;
# (2048, 8192, 4096): 256 blocks of dX, then 512 of dW
@pytest.mark.parametrize("B,I,O", [(4096, 4096, 4096), (2048, 8192, 4096)])
def test_linear_backward_paired_256_tiles_match_separate_launches(gpu, act, accumulate, B, I, O):
    """Where dX and dW both plan to the 256 x 256 tile without split-K, the
    backward runs them in one launch.  Each block computes as in its own
    launch, so dX (with the ReLU mask), dW (also accumulated) and db equal
    separate cnhip_gemm_f32 launches and the column sum bit for bit."""
    print(f"[linear-pair-256] {act} acc={accumulate} B={B} I={I} O={O}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(B + I + O + (7 if accumulate else 0))
    X = torch.randn(B * I, device="cuda", generator=g)
    W = torch.randn(I * O, device="cuda", generator=g) / np.sqrt(I)
    dY = torch.randn(B * O, device="cuda", generator=g)
    aux = torch.relu(torch.randn(B * I, device="cuda", generator=g))
    gW0 = torch.randn(I * O, device="cuda", generator=g) * 1e-3
    gb0 = torch.randn(O, device="cuda", generator=g) * 1e-3
    gW, gb, dX = gW0.clone(), gb0.clone(), torch.empty(B * I, device="cuda")
    if act == "none":
        ops.linear_backward(X, W, dY, gW, gb, dX, B, I, O, True, accumulate)
    else:
        ops.linear_backward_act(X, W, dY, gW, gb, dX, aux, B, I, O, act)
    dXs, gWs, gbs = torch.empty(B * I, device="cuda"), gW0.clone(), gb0.clone()
    ops.gemm(False, True, B, I, O, dY, B, W, I, dXs, B)
    ops.gemm(True, False, I, O, B, X, B, dY, B, gWs, I, beta=1.0 if accumulate else 0.0)
    ops.column_sum(dY, gbs, B, O, accumulate)
    if act == "relu":
        dZ = torch.empty(B * I, device="cuda")
        ops.relu_backward(aux, dXs, dZ)
        dXs = dZ
    torch.cuda.synchronize()
    assert torch.equal(dX, dXs), "dX"
    assert torch.equal(gW, gWs), "grad_W"
    assert torch.equal(gb, gbs), "grad_b"


@pytest.mark.parametrize("act", ["relu", "gelu", "residual"])
@pytest.mark.parametrize("B,I,O", [(4096, 1024, 10), (8192, 512, 1), (2048, 2048, 16)])
def test_linear_backward_one_pass_variants_vs_oracle(gpu, oracle, act, B, I, O):
    """cnhip_linear_backward_act at shapes the one-pass few-output backward
    serves (O in 1..16, B % 512 == 0, B*I >= 2^22), with the activation's
    input (or the skip branch's gradient) a tensor distinct from X: ReLU and
    GELU fold act'(aux) into the one pass's dX; the residual takes the one
    pass for dW, db and then dX = dY W^T + G.  Held to the oracle's Linear
    backward followed by the activation backward (or the add) under the
    contraction bar; the accumulated dW, db start from nonzero values."""
    print(f"[linear-one-pass] {act} B={B} I={I} O={O}", flush=True)
    rng = np.random.default_rng(B + 3 * I + O)
    X, W, dY = rnd(rng, B * I), rnd(rng, I * O, 1 / np.sqrt(I)), rnd(rng, B * O, 0.05)
    aux = rnd(rng, B * I)  # ReLU output / GELU input / skip-branch gradient
    if act == "relu":
        aux = np.maximum(aux, 0)
    gW0, gb0 = rnd(rng, I * O, 1e-3), rnd(rng, O, 1e-3)
    gW, gb, dX = dev(gW0), dev(gb0), torch.empty(B * I, device="cuda")
    ops.linear_backward_act(dev(X), dev(W), dev(dY), gW, gb, dX, dev(aux), B, I, O, act,
                            accumulate=True)
    rgW, rgb, rdL = gW0.copy(), gb0.copy(), np.zeros(B * I, np.float32)
    oracle.cnref_linear_backward(fp(X), fp(W), fp(dY), fp(rgW), fp(rgb), fp(rdL), B, I, O, 1, 1)
    rdX = np.zeros_like(rdL)
    if act == "relu":
        oracle.cnref_relu_backward(fp(aux), fp(rdL), fp(rdX), rdX.size)
    elif act == "gelu":
        oracle.cnref_gelu_backward(fp(aux), fp(rdL), fp(rdX), rdX.size)
    else:
        oracle.cnref_add(fp(rdL), fp(aux), fp(rdX), rdX.size)
    mag_dx = gemm_mag(oracle, 0, 1, B, I, O, dY, B, W, I, B)
    if act == "gelu":  # the contraction's rounding carried through gelu'(aux), |gelu'| <= 1.13
        mag_dx = mag_dx * 1.13
    elif act == "relu":
        mag_dx = mag_dx * (aux > 0)
    mags = {"grad_W": gemm_mag(oracle, 1, 0, I, O, B, X, B, dY, B, I),
            "grad_b": gemm_mag(oracle, 1, 0, 1, O, B, np.ones(B, np.float32), B, dY, B, 1),
            "dX": mag_dx}
    for got, want, name in [(host(gW), rgW, "grad_W"), (host(gb), rgb, "grad_b"), (host(dX), rdX, "dX")]:
        ok, msg = close_mag(got, want, mags[name], RTOL, ATOL)
        assert ok, f"{act} {name}: {msg}"


@pytest.mark.parametrize("B,I,O", [(64, 48, 40), (8192, 2048, 512), (37, 130, 19), (512, 4096, 64)])
def test_linear_fused_residual_matches_unfused(gpu, B, I, O):
    """Y = X W + b + R and dX = dY W^T + G in the GEMM epilogue equal the
    separate Linear call and cnhip_add bit for bit (also through the split-K
    reduce, which the (512, 4096, 64) backward's K = 64 / forward K = 4096
    shapes take)."""
    print(f"[linear-residual] B={B} I={I} O={O}", flush=True)
    rng = np.random.default_rng(B * 3 + I + O)
    X, W, b = dev(rnd(rng, B * I)), dev(rnd(rng, I * O, 1 / np.sqrt(I))), dev(rnd(rng, O, 0.1))
    R = dev(rnd(rng, B * O))
    Y = torch.empty(B * O, device="cuda")
    ops.linear_forward_act(X, W, b, Y, R, B, I, O, "residual")
    Yl, Yu = torch.empty(B * O, device="cuda"), torch.empty(B * O, device="cuda")
    ops.linear_forward(X, W, b, Yl, B, I, O)
    ops.add(Yl, R, Yu)
    np.testing.assert_array_equal(host(Y), host(Yu))
    dY, G = dev(rnd(rng, B * O)), dev(rnd(rng, B * I))
    gW, gb, dX = torch.empty(I * O, device="cuda"), torch.empty(O, device="cuda"), torch.empty(B * I, device="cuda")
    ops.linear_backward_act(X, W, dY, gW, gb, dX, G, B, I, O, "residual")
    gWu, gbu, dXl, dXu = (torch.empty(I * O, device="cuda"), torch.empty(O, device="cuda"),
                          torch.empty(B * I, device="cuda"), torch.empty(B * I, device="cuda"))
    ops.linear_backward(X, W, dY, gWu, gbu, dXl, B, I, O, True, False)
    ops.add(dXl, G, dXu)
    np.testing.assert_array_equal(host(dX), host(dXu))
    np.testing.assert_array_equal(host(gW), host(gWu))
    np.testing.assert_array_equal(host(gb), host(gbu))


@pytest.mark.parametrize("n", [1, 512, 1000, 4097, 65536])
@pytest.mark.parametrize("red_f,red_b", [(0, 0), (1, 1), (0, 1)])
def test_sigmoid_bce_head_matches_separate_kernels(gpu, n, red_f, red_b):
    """cnhip_sigmoid_bce_head against cnhip_sigmoid_forward + cnhip_bce_forward
    + cnhip_bce_backward + cnhip_sigmoid_backward: every output bit-identical
    (reduction codes 0 mean, 1 sum; "none" uses mean forward, sum backward)."""
    from cppnet_amd import _capi
    lib = _capi.load()
    print(f"[ops] sigmoid+bce head n={n} red={red_f},{red_b}", flush=True)
    rng = np.random.default_rng(n)
    z = torch.from_numpy((rng.standard_normal(n) * 4).astype(np.float32)).cuda()
    t = torch.from_numpy((rng.uniform(size=n) < 0.5).astype(np.float32)).cuda()
    s = torch.cuda.current_stream().cuda_stream
    p1, g1, dz1 = (torch.empty(n, device="cuda") for _ in range(3))
    l1 = torch.empty(1, device="cuda")
    assert lib.cnhip_sigmoid_forward(z.data_ptr(), p1.data_ptr(), n, s) == 0
    assert lib.cnhip_bce_forward(p1.data_ptr(), t.data_ptr(), l1.data_ptr(), n, red_f, s) == 0
    assert lib.cnhip_bce_backward(p1.data_ptr(), t.data_ptr(), g1.data_ptr(), n, red_b, s) == 0
    assert lib.cnhip_sigmoid_backward(p1.data_ptr(), g1.data_ptr(), dz1.data_ptr(), n, s) == 0
    p2, dz2 = torch.empty(n, device="cuda"), torch.empty(n, device="cuda")
    l2 = torch.empty(1, device="cuda")
    assert lib.cnhip_sigmoid_bce_head(z.data_ptr(), t.data_ptr(), p2.data_ptr(), l2.data_ptr(),
                                      dz2.data_ptr(), n, red_f, red_b, s) == 0
    torch.cuda.synchronize()
    for a, b, name in [(p1, p2, "p"), (l1, l2, "loss"), (dz1, dz2, "dz")]:
        assert torch.equal(a.view(torch.int32), b.view(torch.int32)), name


@pytest.mark.parametrize("B,C", [(1, 1), (32, 4), (256, 10), (200, 7), (64, 16), (100, 17), (256, 32),
                                 (77, 33), (257, 10), (4096, 10), (300, 40), (600, 32)])
@pytest.mark.parametrize("red", [0, 1])
def test_softmax_ce_head_matches_separate_kernels(gpu, B, C, red):
    """cnhip_softmax_ce_head against cnhip_softmax_ce_forward +
    cnhip_softmax_ce_backward: softmax, loss and gradient bit-identical (one
    launch up to 256 rows; beyond, per-block rows with the gradient for up
    to 32 classes, the separate backward kernel for more)."""
    from cppnet_amd import _capi
    lib = _capi.load()
    print(f"[ops] softmax-CE head B={B} C={C} red={red}", flush=True)
    rng = np.random.default_rng(B * 31 + C)
    z = torch.from_numpy((rng.standard_normal(B * C) * 3).astype(np.float32)).cuda()
    lab = rng.integers(0, C, B)
    t_np = np.zeros((C, B), np.float32)
    t_np[lab, np.arange(B)] = 1.0
    t = torch.from_numpy(t_np.ravel()).cuda()
    s = torch.cuda.current_stream().cuda_stream
    sm1, g1, l1 = torch.empty(B * C, device="cuda"), torch.empty(B * C, device="cuda"), torch.empty(1, device="cuda")
    assert lib.cnhip_softmax_ce_forward(z.data_ptr(), t.data_ptr(), sm1.data_ptr(), l1.data_ptr(), B, C, red, s) == 0
    assert lib.cnhip_softmax_ce_backward(sm1.data_ptr(), t.data_ptr(), g1.data_ptr(), B, C, red, s) == 0
    sm2, g2, l2 = torch.empty(B * C, device="cuda"), torch.empty(B * C, device="cuda"), torch.empty(1, device="cuda")
    assert lib.cnhip_softmax_ce_head(z.data_ptr(), t.data_ptr(), sm2.data_ptr(), l2.data_ptr(), g2.data_ptr(),
                                     B, C, red, s) == 0
    torch.cuda.synchronize()
    for a, b, name in [(sm1, sm2, "softmax"), (l1, l2, "loss"), (g1, g2, "grad")]:
        assert torch.equal(a.view(torch.int32), b.view(torch.int32)), name
