"""cnhip_linear_backward_act_noalloc against cnhip_linear_backward_act, through
the C ABI: the same kernels with their workspace in the library's fixed
32 MiB device array, so the results must be equal bit for bit.  Each case
makes two no-allocation calls in a row, the second with a smaller input, so
the second runs over the first's leftover workspace contents.  The paths
covered are the ones that use a workspace: the split-K dW GEMM, the one-pass
head backward (its row-chunk partials, with and without a separate dX GEMM
after it), plus a shape that needs none; a shape whose workspace would not
fit is refused before anything runs."""
import numpy as np
import pytest
import torch

from cppnet_amd import _capi, ops

pytestmark = pytest.mark.gpu

# (B, I, O, act, accumulate): first call, then a smaller second call
CASES = {
    # dW = X^T dY with K = B: 64 x 64 tiles split 8 ways (8 MiB of partials)
    "splitk": ((8192, 512, 512, "none", False), (4096, 512, 256, "none", False)),
    # one-pass head backward (O = 10): 8, then 2 row chunks of partials
    "head_relu": ((4096, 4096, 10, "relu", False), (1024, 4096, 10, "relu", False)),
    # one-pass dW / db, then the dX GEMM with the residual sum in its epilogue
    "head_residual": ((4096, 1024, 16, "residual", True), (1024, 4096, 8, "residual", True)),
    # SIMT small GEMMs: no workspace at all
    "small": ((64, 48, 40, "gelu", False), (37, 30, 19, "gelu", False)),
}


def _inputs(rng, B, I, O):
    f = lambda n, s=1.0: torch.from_numpy((rng.standard_normal(n) * s).astype(np.float32)).cuda()  # noqa: E731
    return dict(X=f(B * I), W=f(I * O, 1 / np.sqrt(I)), dY=f(B * O), aux=f(B * I), gW0=f(I * O), gb0=f(O))


def _run(fn, t, B, I, O, act, acc):
    gW, gb = t["gW0"].clone(), t["gb0"].clone()
    dX = torch.full((B * I,), float("nan"), device="cuda")
    aux = t["aux"] if act != "none" else None
    fn(t["X"], t["W"], t["dY"], gW, gb, dX, aux, B, I, O, act, True, acc)
    torch.cuda.synchronize()
    return gW.cpu().numpy(), gb.cpu().numpy(), dX.cpu().numpy()


@pytest.mark.parametrize("case", sorted(CASES))
def test_noalloc_matches_linear_backward_act(gpu, case):
    rng = np.random.default_rng(sorted(CASES).index(case) + 70)
    for call, (B, I, O, act, acc) in enumerate(CASES[case]):
        print(f"[noalloc] {case} call {call}: B={B} I={I} O={O} act={act} accumulate={acc}", flush=True)
        t = _inputs(rng, B, I, O)
        want = _run(ops.linear_backward_act, t, B, I, O, act, acc)
        got = _run(ops.linear_backward_act_noalloc, t, B, I, O, act, acc)
        for name, a, b in zip(("grad_W", "grad_b", "dX"), got, want):
            assert not np.isnan(b).any(), f"{name}: the allocating entry point left NaNs"
            np.testing.assert_array_equal(a, b, err_msg=f"{case} call {call}: {name}")


def test_noalloc_refuses_workspace_beyond_its_array(gpu):
    """The one-pass head backward at B = 129 x 512 rows, I = 4096, O = 16 needs
    258 row chunks of 256 x (4096 x 16 + 16) floats = 67.7 MB > 32 MiB of partials: the
    call fails with CNHIP_EINVAL and a message, and leaves every output as it
    was.  The buffers are full size, so even a call that ran would stay in
    bounds."""
    B, I, O = 129 * 512, 4096, 16
    print(f"[noalloc] refusal: B={B} I={I} O={O}", flush=True)
    X = torch.ones(B * I, device="cuda")
    W = torch.ones(I * O, device="cuda")
    dY = torch.ones(B * O, device="cuda")
    gW = torch.full((I * O,), 7.0, device="cuda")
    gb = torch.full((O,), 7.0, device="cuda")
    dX = torch.full((B * I,), 7.0, device="cuda")
    with pytest.raises(_capi.CnhipError, match="fixed device workspace"):
        ops.linear_backward_act_noalloc(X, W, dY, gW, gb, dX, None, B, I, O, "none")
    torch.cuda.synchronize()
    for name, t in (("grad_W", gW), ("grad_b", gb), ("dX", dX)):
        assert bool((t == 7.0).all()), f"{name} was written by a refused call"
    del X, dX
    torch.cuda.empty_cache()
