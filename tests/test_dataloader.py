"""DataLoader host logic (no GPU): the reference's own checks
(tests/utils/test_dataloader.cpp:34-107: construction, num_batches with and
without drop_last, batch count and dimensions, the short last batch, full
coverage in order without shuffle, re-iteration after reset, a shuffle that
loses nothing) plus what they leave open: every batch holds exactly the rows
that the epoch's index order names, and a seed fixes that order."""
import numpy as np
import pytest

from cppnet_amd import trainer


def _dataset(n, f, l, rng=None):
    if rng is None:  # the reference test's data: feature (i, j) = i*f + j, label i
        X = np.arange(n * f, dtype=np.float32).reshape(n, f)
        Y = np.arange(n, dtype=np.float32).reshape(n, 1).repeat(l, axis=1)
    else:
        X = rng.standard_normal((n, f)).astype(np.float32)
        Y = rng.standard_normal((n, l)).astype(np.float32)
    return X, Y


def _loader(X, Y, batch, shuffle=True, drop_last=False, seed=0):
    n, f = X.shape
    return trainer.Loader(X.ravel(order="F"), Y.ravel(order="F"), n, f, Y.shape[1], batch, shuffle,
                          drop_last, seed)


def test_reference_cases():
    X, Y = _dataset(10, 3, 1)
    assert _loader(X, Y, 4).num_batches == 3
    assert _loader(X, Y, 4, drop_last=True).num_batches == 2
    ld = _loader(X, Y, 3)
    assert ld.num_batches == 4
    sizes = [ld.host_batch(k)[2] for k in range(ld.num_batches)]
    assert sizes == [3, 3, 3, 1]
    ld = _loader(X, Y, 4, shuffle=False)
    x, y, bs = ld.host_batch(0)
    assert bs == 4 and x.size == 4 * 3 and y.size == 4
    assert ld.host_batch(2)[2] == 2
    x, y, bs = _loader(X, Y, 10, shuffle=False).host_batch(0)
    np.testing.assert_array_equal(y, np.arange(10, dtype=np.float32))
    np.testing.assert_array_equal(x.reshape(3, 10).T, X)
    ld = _loader(X, Y, 3)
    n1 = ld.num_batches
    ld.reset()
    assert ld.num_batches == n1
    total = sum(ld.host_batch(k)[1].sum() for k in range(ld.num_batches))
    assert total == pytest.approx(45.0)
    with pytest.raises(Exception, match="batch_size must be > 0"):
        _loader(X, Y, 0)


@pytest.mark.parametrize("n,f,l,batch,drop", [(10, 3, 1, 3, False), (257, 37, 3, 64, False),
                                              (257, 37, 3, 64, True), (64, 5, 2, 64, False)])
def test_batches_follow_the_epoch_order(n, f, l, batch, drop):
    X, Y = _dataset(n, f, l, np.random.default_rng(n + f))
    ld = _loader(X, Y, batch, drop_last=drop, seed=7)
    for epoch in range(2):
        idx = ld.indices()
        assert sorted(idx.tolist()) == list(range(n))
        for k in range(ld.num_batches):
            x, y, bs = ld.host_batch(k)
            rows = idx[k * batch:k * batch + bs]
            np.testing.assert_array_equal(x.reshape(f, bs).T, X[rows])
            np.testing.assert_array_equal(y.reshape(l, bs).T, Y[rows])
        ld.reset()
        assert epoch == 1 or not np.array_equal(ld.indices(), idx)


def test_seed_fixes_the_order():
    X, Y = _dataset(100, 2, 1)
    a, b, c = _loader(X, Y, 10, seed=3), _loader(X, Y, 10, seed=3), _loader(X, Y, 10, seed=4)
    np.testing.assert_array_equal(a.indices(), b.indices())
    assert not np.array_equal(a.indices(), c.indices())
    np.testing.assert_array_equal(_loader(X, Y, 10, shuffle=False).indices(), np.arange(100))


def test_errors_are_reported_not_raised_through():
    """Bad arguments come back as a status and a message (no GPU needed)."""
    import ctypes as C
    X, Y = _dataset(10, 3, 1)
    ld = _loader(X, Y, 4, shuffle=False)
    with pytest.raises(Exception, match="out of range"):
        ld.host_batch(3)
    with pytest.raises(Exception, match="out of range"):
        ld.host_batch(-1)
    lib = trainer.load()
    h = C.c_void_p()
    x = np.zeros(30, np.float32)
    assert lib.cnt_loader_create(C.byref(h), x.ctypes.data, x.ctypes.data, 10, 0, 1, 4, 1, 0, 0) != 0
    assert "shape" in lib.cnt_last_error().decode()
    assert lib.cnt_loader_create(None, x.ctypes.data, x.ctypes.data, 10, 3, 1, 4, 1, 0, 0) != 0
    n = C.c_int64()
    assert lib.cnt_loader_num_batches(None, C.byref(n)) != 0
    assert "NULL loader" in lib.cnt_last_error().decode()
