"""CPU-side checks of the host layer and trainer front end (no GPU):
configuration shapes, synthetic data layout and error paths that the C++
classes raise before touching a device."""
import ctypes as C

import numpy as np
import pytest

from cppnet_amd import trainer


def test_config_shapes_match_baseline():
    c1, c2 = trainer.mlp_config(1), trainer.mlp_config(2)
    assert (c1.sizes, c1.batch, c1.loss, c1.out_act) == ([30, 64, 1], 512, "bce", "sigmoid")
    assert (c2.sizes, c2.batch, c2.loss) == ([1024, 4096, 4096, 10], 4096, "softmax_ce")
    n2 = sum(i * o + o for i, o in zip(c2.sizes[:-1], c2.sizes[1:]))
    assert n2 == 21_020_682  # config 2: 1024*4096 + 4096 + 4096*4096 + 4096 + 4096*10 + 10
    n1 = sum(i * o + o for i, o in zip(c1.sizes[:-1], c1.sizes[1:]))
    assert n1 == 2_049


def test_synthetic_targets_are_colmajor_one_hot():
    cfg = trainer.mlp_config(2, batch=64)
    params, X, Y = trainer.synthetic_mlp(cfg, np.random.default_rng(0))
    Yl = Y.reshape(10, 64).T  # logical [B, C]
    assert np.all(Yl.sum(1) == 1.0) and set(np.unique(Yl)) == {0.0, 1.0}
    lim = np.sqrt(6 / (1024 + 4096))
    assert np.abs(params[0]).max() <= lim and np.all(params[1] == 0)


def test_create_rejects_bad_arguments_without_gpu():
    lib = trainer.load()
    h = C.c_void_p()
    sizes = (C.c_int64 * 2)(4, 2)
    st = lib.cnt_mlp_create(C.byref(h), 0, sizes, 1, 0, 1, 8, 1e-3, 0.9, 0.999, 1e-8, 0)
    assert st != 0 and b"at least one" in lib.cnt_last_error()
    st = lib.cnt_mlp_create(C.byref(h), 1, sizes, 1, 0, 1, 0, 1e-3, 0.9, 0.999, 1e-8, 0)
    assert st != 0 and b"batch" in lib.cnt_last_error()
    st = lib.cnt_step(None, None)
    assert st != 0 and b"NULL session" in lib.cnt_last_error()
