"""DataLoader device staging (cnt_loader_*): the resident gather kernel and the
page-locked double-buffered stream deliver, batch for batch and bit for bit,
what the host iterator (the reference's get_batch, checked on the CPU in
tests/test_dataloader.py) yields, over several epochs with reshuffles; and a
session trained from the loader steps exactly as one fed the same batches
with cnt_set_batch."""
import numpy as np
import pytest
import torch

from cppnet_amd import trainer

pytestmark = pytest.mark.gpu


def _data(n, f, l, seed):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((n, f)).astype(np.float32)
    Y = rng.standard_normal((n, l)).astype(np.float32)
    return X, Y


# (n, f, l, batch, drop_last): scalar and float4 gather paths, short last
# batches, one batch, more than 2^16 values per batch row tile grid
CASES = [(257, 37, 3, 64, False), (4096, 1024, 10, 512, True), (1000, 64, 1, 1000, False),
         (300, 8, 2, 7, False), (130, 96, 4, 64, True)]


@pytest.mark.parametrize("mode", ["resident", "stream"])
@pytest.mark.parametrize("n,f,l,batch,drop", CASES)
def test_device_batches_match_host(gpu, mode, n, f, l, batch, drop):
    print(f"[loader] {mode} n={n} f={f} l={l} batch={batch} drop_last={drop}", flush=True)
    X, Y = _data(n, f, l, n + f)
    ld = trainer.Loader(X.ravel(order="F"), Y.ravel(order="F"), n, f, l, batch, True, drop, seed=5)
    ld.to_device(mode)
    xb = torch.empty(batch * f, device="cuda")
    yb = torch.empty(batch * l, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    for epoch in range(3):
        for k in range(ld.num_batches):
            hx, hy, hbs = ld.host_batch(k)
            bs = ld.next(xb.data_ptr(), yb.data_ptr(), stream)
            assert bs == hbs, f"epoch {epoch} batch {k}: size {bs} vs {hbs}"
            torch.cuda.synchronize()
            np.testing.assert_array_equal(xb[:bs * f].cpu().numpy(), hx)
            np.testing.assert_array_equal(yb[:bs * l].cpu().numpy(), hy)
        assert ld.next(xb.data_ptr(), yb.data_ptr(), stream) == 0  # end of the epoch
        ld.reset()
    ld.close()


@pytest.mark.parametrize("mode", ["resident", "stream"])
def test_training_from_loader_matches_set_batch(gpu, mode):
    cfg = trainer.MLPConfig("MLP 40-64-5", [40, 64, 5], "relu", "none", "mse", 32)
    print(f"[loader] training {mode}", flush=True)
    n = 32 * 6
    X, Y = _data(n, 40, 5, 9)
    params = trainer.synthetic_mlp(cfg, np.random.default_rng(1))[0]
    ld = trainer.Loader(X.ravel(order="F"), Y.ravel(order="F"), n, 40, 5, 32, True, True, seed=11)
    ld.to_device(mode)
    a, b = trainer.Session(cfg), trainer.Session(cfg)
    a.set_params(params)
    b.set_params(params)
    for epoch in range(2):
        for k in range(ld.num_batches):
            hx, hy, _ = ld.host_batch(k)
            assert ld.next_batch(a) == 32
            b.set_batch(hx, hy)
            la, lb = a.step(), b.step()
            assert np.float32(la).view(np.uint32) == np.float32(lb).view(np.uint32), (
                f"epoch {epoch} batch {k}: {la!r} vs {lb!r}")
        assert ld.next_batch(a) == 0
        ld.reset()
    for pa, pb in zip(a.get_params(), b.get_params()):
        np.testing.assert_array_equal(pa, pb)
    a.close()
    b.close()
    ld.close()


def test_session_batch_mismatch_is_refused(gpu):
    cfg = trainer.MLPConfig("MLP 40-8-5", [40, 8, 5], "relu", "none", "mse", 32)
    X, Y = _data(50, 40, 5, 2)
    ld = trainer.Loader(X.ravel(order="F"), Y.ravel(order="F"), 50, 40, 5, 32, False, False, seed=1)
    ld.to_device("resident")
    s = trainer.Session(cfg)
    assert ld.next_batch(s) == 32
    with pytest.raises(Exception, match="drop_last"):
        ld.next_batch(s)  # the short last batch (18) does not fit a batch-32 session
    s.close()
    ld.close()


@pytest.mark.parametrize("mode", ["resident", "stream"])
def test_queued_epoch_then_reset(gpu, mode):
    """A whole epoch of batches queued on a non-blocking stream behind ~5 ms of
    other work, then reset() (a new permutation, uploaded at once) and the
    next epoch queued too, before any gather has run: every batch must still
    be gathered with its own epoch's order.  Then to_device() again (which
    frees the staged dataset) with the second epoch still queued, right after
    the reset started the next epoch's staging worker."""
    from cppnet_amd import _capi
    n, f, l, batch = 2048, 96, 4, 128
    print(f"[loader] {mode}: queued epochs across reset", flush=True)
    X, Y = _data(n, f, l, 77)
    ld = trainer.Loader(X.ravel(order="F"), Y.ravel(order="F"), n, f, l, batch, True, True, seed=3)
    ld.to_device(mode)
    lib = _capi.load()
    st = _capi.C.c_void_p()
    assert lib.cnhip_stream_create(_capi.C.byref(st)) == 0
    stream = st.value
    M = 4096
    A = torch.randn(M * M, device="cuda")
    Cm = torch.empty(M * M, device="cuda")
    torch.cuda.synchronize()
    for _ in range(12):  # ~5 ms queued ahead of the gathers
        assert lib.cnhip_gemm_f32(0, 0, M, M, M, 1.0, A.data_ptr(), M, A.data_ptr(), M, 0.0, Cm.data_ptr(), M,
                                  None, 0, stream) == 0
    nb = ld.num_batches
    epochs = []
    for epoch in range(2):
        host = [ld.host_batch(k) for k in range(nb)]
        xb = torch.empty((nb, batch * f), device="cuda")
        yb = torch.empty((nb, batch * l), device="cuda")
        for k in range(nb):
            assert ld.next(xb[k].data_ptr(), yb[k].data_ptr(), stream) == batch
        epochs.append((host, xb, yb))
        ld.reset()
    ld.to_device(mode)  # frees the staged copy while the second epoch may still be queued
    assert lib.cnhip_stream_synchronize(stream) == 0
    for epoch, (host, xb, yb) in enumerate(epochs):
        for k, (hx, hy, _) in enumerate(host):
            np.testing.assert_array_equal(xb[k].cpu().numpy(), hx, err_msg=f"epoch {epoch} batch {k}")
            np.testing.assert_array_equal(yb[k].cpu().numpy(), hy, err_msg=f"epoch {epoch} batch {k}")
    assert not np.array_equal(epochs[0][0][0][0], epochs[1][0][0][0])  # the orders differ
    ld.close()
    assert lib.cnhip_stream_destroy(stream) == 0
