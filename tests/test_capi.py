"""CPU-only checks of the C-ABI library: it loads, exports every symbol its
headers declare, and its argument validation returns the documented status
codes (validation runs before any HIP call, so no GPU is needed)."""
import ctypes as C
from pathlib import Path

import pytest

from cppnet_amd import _capi

ROOT = Path(__file__).resolve().parent.parent


def test_library_exports_every_declared_symbol():
    lib = _capi.load()
    declared = _capi.header_symbols(ROOT / "include" / "cnhip.h")
    assert len(declared) >= 30
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, f"declared in cnhip.h but not exported: {missing}"
    unbound = [s for s in declared if s not in _capi.SIGNATURES]
    assert not unbound, f"no ctypes signature for: {unbound}"


def test_trainer_library_exports_every_declared_symbol():
    from cppnet_amd import trainer
    lib = trainer.load()
    declared = _capi.header_symbols(ROOT / "include" / "cppnet_train.h")
    assert declared
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, f"declared in cppnet_train.h but not exported: {missing}"


def test_version_and_device_count_without_gpu():
    lib = _capi.load()
    assert lib.cnhip_version().decode().startswith("cnhip")
    assert lib.cnhip_device_count() >= 0


def _status_and_error(fn, *args):
    st = fn(*args)
    return st, _capi.load().cnhip_last_error().decode()


def test_gemm_rejects_bad_arguments():
    lib = _capi.load()
    st, msg = _status_and_error(lib.cnhip_gemm_f32, 0, 0, -1, 4, 4, 1.0, None, 1, None, 1, 0.0,
                                None, 1, None, 0, None)
    assert st == 1 and "negative" in msg
    dummy = C.c_void_p(16)  # never dereferenced: validation fails first
    st, msg = _status_and_error(lib.cnhip_gemm_f32, 0, 0, 8, 4, 4, 1.0, dummy, 8, dummy, 4, 0.0,
                                dummy, 4, None, 0, None)
    assert st == 1 and "ldc" in msg
    st, msg = _status_and_error(lib.cnhip_gemm_f32, 0, 0, 8, 4, 4, 1.0, dummy, 8, dummy, 4, 0.0,
                                dummy, 8, None, 7, None)
    assert st == 1 and "epilogue" in msg
    st, msg = _status_and_error(lib.cnhip_gemm_f32, 1, 0, 8, 4, 4, 1.0, dummy, 3, dummy, 4, 0.0,
                                dummy, 8, None, 0, None)
    assert st == 1 and "lda" in msg


def test_losses_reject_bad_reduction_and_empty_input():
    lib = _capi.load()
    d = C.c_void_p(16)
    st, msg = _status_and_error(lib.cnhip_bce_forward, d, d, d, 4, 5, None)
    assert st == 1 and "reduction" in msg
    st, msg = _status_and_error(lib.cnhip_softmax_ce_forward, d, d, d, d, 0, 3, 0, None)
    assert st == 1 and "empty" in msg
    st, msg = _status_and_error(lib.cnhip_mse_backward, None, d, d, 3, 0, None)
    assert st == 1 and "NULL" in msg


def test_adam_rejects_zero_bias_correction_and_too_many_tensors():
    lib = _capi.load()
    d = C.c_void_p(16)
    st, msg = _status_and_error(lib.cnhip_adam_step, d, d, d, d, 4, 1e-3, 0.9, 0.999, 1e-8, 0.0,
                                0.1, None)
    assert st == 1 and "bias correction" in msg
    st, msg = _status_and_error(lib.cnhip_adam_step_multi, 65, None, None, None, None, None, None,
                                None, 1e-3, 0.9, 0.999, 1e-8, None)
    assert st == 1 and "count" in msg


def test_linear_rejects_bad_shapes():
    lib = _capi.load()
    d = C.c_void_p(16)
    st, msg = _status_and_error(lib.cnhip_linear_forward, d, d, None, d, 4, 0, 3, None)
    assert st == 1 and "bad shape" in msg
    st, msg = _status_and_error(lib.cnhip_linear_backward, d, d, d, None, None, None, 4, 2, 3, 1,
                                1, None)
    assert st == 1 and "grad_W" in msg
    # the no-allocation variant checks shape and activation before any HIP call
    st, msg = _status_and_error(lib.cnhip_linear_backward_act_noalloc, d, d, d, d, d, d, None, -1, 2, 3, 1,
                                0, 0, None)
    assert st == 1 and "bad shape" in msg
    st, msg = _status_and_error(lib.cnhip_linear_backward_act_noalloc, d, d, d, d, d, d, None, 4, 2, 3, 1,
                                0, 9, None)
    assert st == 1 and "bad activation" in msg


def test_ops_refuse_host_tensors():
    import torch
    from cppnet_amd import ops
    x = torch.zeros(4)
    with pytest.raises(TypeError, match="device tensor"):
        ops.relu_forward(x, x)


def test_graph_entry_points_validate_without_gpu():
    lib = _capi.load()
    st, msg = _status_and_error(lib.cnhip_graph_begin_capture, None)
    assert st == 1 and "default stream" in msg
    st, msg = _status_and_error(lib.cnhip_graph_launch, None, None)
    assert st == 1 and "NULL graph" in msg
    assert lib.cnhip_graph_destroy(None) == 0
