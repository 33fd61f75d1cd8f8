"""CPU oracle (test infrastructure): loader of oracle/liboracle.so and small
helpers for Eigen ColMajor data.  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg use it; the product (cppnet_amd) never does."""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
ORACLE_SO = ORACLE_DIR / "liboracle.so"

_f = C.POINTER(C.c_float)
_i = C.POINTER(C.c_int32)
i64, f32, i32 = C.c_int64, C.c_float, C.c_int
_SIGS = {
    "cnref_set_threads": (None, [i32]),
    "cnref_get_threads": (i32, []),
    "cnref_set_accumulate_double": (None, [i32]),
    "cnref_set_sum_order": (None, [i32]),
    "cnref_set_cpu_loops": (None, [i32]),
    "cnref_get_cpu_loops": (i32, []),
    "cnref_set_trace": (None, [i32, _f]),
    "cnref_trace": (_f, [i32]),
    "cnref_gemm_f32": (None, [i32, i32, i64, i64, i64, f32, _f, i64, _f, i64, f32, _f, i64, _f,
                              i32]),
    "cnref_linear_forward": (None, [_f, _f, _f, _f, i64, i64, i64]),
    "cnref_linear_backward": (None, [_f, _f, _f, _f, _f, _f, i64, i64, i64, i32, i32]),
    "cnref_column_sum": (None, [_f, _f, i64, i64, i32]),
    "cnref_add": (None, [_f, _f, _f, i64]),
    "cnref_residual_forward": (None, [i32, C.POINTER(i64), C.POINTER(_f), C.POINTER(_f), _f, _f,
                                      C.POINTER(_f), _f, i64]),
    "cnref_residual_backward": (None, [i32, C.POINTER(i64), C.POINTER(_f), _f, _f, C.POINTER(_f), _f,
                                       C.POINTER(_f), C.POINTER(_f), _f, _f, i64]),
    "cnref_relu_forward": (None, [_f, _f, i64]),
    "cnref_leaky_relu_forward": (None, [_f, _f, i64, f32]),
    "cnref_leaky_relu_backward": (None, [_f, _f, _f, i64, f32]),
    "cnref_softmax_forward": (None, [_f, _f, i64, i64]),
    "cnref_softmax_backward": (None, [_f, _f, _f, i64, i64]),
    "cnref_cce_forward": (f32, [_f, _f, _f, _f, i64, i64, i32, f32, i32]),
    "cnref_cce_backward": (None, [_f, _f, _f, i64, i64, i32, i32]),
    "cnref_mae_forward": (f32, [_f, _f, i64, i32]),
    "cnref_mae_backward": (None, [_f, _f, _f, i64, i32]),
    "cnref_huber_forward": (f32, [_f, _f, i64, f32, i32]),
    "cnref_huber_backward": (None, [_f, _f, _f, i64, f32, i32]),
    "cnref_sgd_step": (None, [_f, _f, i64, f32]),
    "cnref_momentum_step": (None, [_f, _f, _f, i64, f32, f32]),
    "cnref_adagrad_step": (None, [_f, _f, _f, i64, f32, f32]),
    "cnref_rmsprop_step": (None, [_f, _f, _f, i64, f32, f32, f32]),
    "cnref_dropout_apply": (None, [_f, _f, _f, i64, f32]),
    "cnref_global_avgpool_forward": (None, [_f, _f, i64, i64, i64, i64]),
    "cnref_global_avgpool_backward": (None, [_f, _f, i64, i64, i64, i64]),
    "cnref_global_maxpool_forward": (None, [_f, _f, _i, _i, i64, i64, i64, i64]),
    "cnref_global_maxpool_backward": (None, [_f, _i, _i, _f, i64, i64, i64, i64]),
    "cnref_rnn_forward": (None, [_f, _f, _f, _f, _f, i64, i64, i64, i64]),
    "cnref_rnn_backward": (None, [_f] * 9 + [i64] * 4),
    "cnref_relu_backward": (None, [_f, _f, _f, i64]),
    "cnref_sigmoid_forward": (None, [_f, _f, i64]),
    "cnref_sigmoid_backward": (None, [_f, _f, _f, i64]),
    "cnref_tanh_forward": (None, [_f, _f, i64]),
    "cnref_tanh_backward": (None, [_f, _f, _f, i64]),
    "cnref_bce_forward": (f32, [_f, _f, i64, i32]),
    "cnref_bce_backward": (None, [_f, _f, _f, i64, i32]),
    "cnref_mse_forward": (f32, [_f, _f, i64, i32]),
    "cnref_mse_backward": (None, [_f, _f, _f, i64, i32]),
    "cnref_softmax_ce_forward": (f32, [_f, _f, _f, i64, i64, i32]),
    "cnref_softmax_ce_backward": (None, [_f, _f, _f, i64, i64, i32]),
    "cnref_conv2d_forward": (None, [_f, _f, _f, _f] + [i64] * 8),
    "cnref_conv2d_backward": (None, [_f, _f, _f, _f, _f, _f] + [i64] * 8),
    "cnref_maxpool2d_forward": (None, [_f, _f, _i, i64, i64, i64, i64, i64, i64]),
    "cnref_maxpool2d_backward": (None, [_f, _i, _f, i64, i64, i64, i64, i64, i64]),
    "cnref_lstm_forward": (None, [_f] * 8 + [i64] * 4),
    "cnref_lstm_backward": (None, [_f] * 12 + [i64] * 4),
    "cnref_gru_forward": (None, [_f] * 7 + [i64] * 4),
    "cnref_gru_backward": (None, [_f] * 11 + [i64] * 4),
    "cnref_embedding_forward": (i32, [_i, _f, _f, i64, i64, i64, i64]),
    "cnref_embedding_backward": (None, [_i, _f, _f, i64, i64, i64, i64]),
    "cnref_mha_forward": (None, [_f] * 9 + [i64] * 4),
    "cnref_mha_backward": (None, [_f] * 14 + [i64] * 4),
    "cnref_batchnorm_forward": (None, [_f] * 9 + [i64, i64, f32, f32]),
    "cnref_batchnorm_backward": (None, [_f] * 9 + [i64, i64, f32]),
    "cnref_gelu_forward": (None, [_f, _f, i64]),
    "cnref_gelu_backward": (None, [_f, _f, _f, i64]),
    "cnref_meanpool1d_forward": (None, [_f, _f, i64, i64, i64]),
    "cnref_meanpool1d_backward": (None, [_f, _f, i64, i64, i64]),
    "cnref_adam_step": (None, [_f, _f, _f, _f, i64, f32, f32, f32, f32, f32, f32]),
    "cnref_bias_correction": (f32, [f32, i32]),
}

_lib = None


def load_oracle():
    global _lib
    if _lib is not None:
        return _lib
    if not ORACLE_SO.exists():
        # Build from source (in this container; the GPU box receives the built file).
        subprocess.run(["make", "-C", str(ORACLE_DIR)], check=True, stdout=subprocess.DEVNULL)
    lib = C.CDLL(str(ORACLE_SO))
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def fp(a: np.ndarray | None):
    """float* of a float32 numpy buffer (None -> NULL)."""
    if a is None:
        return None
    assert a.dtype == np.float32 and (a.flags["C_CONTIGUOUS"] or a.flags["F_CONTIGUOUS"])
    return a.ctypes.data_as(_f)


def ip(a: np.ndarray | None):
    """int32* of an int32 numpy buffer (None -> NULL)."""
    if a is None:
        return None
    assert a.dtype == np.int32 and (a.flags["C_CONTIGUOUS"] or a.flags["F_CONTIGUOUS"])
    return a.ctypes.data_as(_i)


def colmajor(rows_logical) -> np.ndarray:
    """Logical [[row0], [row1], ...] -> flat float32 in Eigen ColMajor order."""
    a = np.asarray(rows_logical, dtype=np.float32)
    if a.ndim == 1:
        return a.copy()
    return np.array(a.T, dtype=np.float32, order="C").ravel()


def from_colmajor(flat: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Flat ColMajor buffer -> logical [rows, cols] array."""
    return np.asarray(flat).reshape(cols, rows).T


