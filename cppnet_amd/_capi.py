"""ctypes binding of the C ABI in include/cnhip.h (libcnhip.so).

The library is loaded from cppnet_amd/_lib/.  There is no fallback: if the
HIP library is missing, importing the op wrappers raises, so nothing can run
silently on a CPU path.
"""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIBDIR = PKG / "_lib"
HEADER = PKG.parent / "include" / "cnhip.h"

i64 = C.c_int64
f32 = C.c_float
vp = C.c_void_p
i32 = C.c_int

# name -> (restype, argtypes)
SIGNATURES: dict[str, tuple] = {
    "cnhip_last_error": (C.c_char_p, []),
    "cnhip_version": (C.c_char_p, []),
    "cnhip_device_count": (i32, []),
    "cnhip_set_device": (i32, [i32]),
    "cnhip_malloc": (i32, [C.POINTER(vp), C.c_size_t]),
    "cnhip_free": (i32, [vp]),
    "cnhip_memcpy_async": (i32, [vp, vp, C.c_size_t, i32, vp]),
    "cnhip_memset_async": (i32, [vp, i32, C.c_size_t, vp]),
    "cnhip_stream_create": (i32, [C.POINTER(vp)]),
    "cnhip_stream_destroy": (i32, [vp]),
    "cnhip_stream_synchronize": (i32, [vp]),
    "cnhip_device_synchronize": (i32, []),
    "cnhip_is_device_pointer": (i32, [vp]),
    "cnhip_event_create": (i32, [C.POINTER(vp)]),
    "cnhip_event_destroy": (i32, [vp]),
    "cnhip_event_record": (i32, [vp, vp]),
    "cnhip_event_elapsed_ms": (i32, [C.POINTER(f32), vp, vp]),
    "cnhip_event_synchronize": (i32, [vp]),
    "cnhip_stream_wait_event": (i32, [vp, vp]),
    "cnhip_get_device": (i32, [C.POINTER(i32)]),
    "cnhip_host_alloc": (i32, [C.POINTER(vp), C.c_size_t]),
    "cnhip_host_free": (i32, [vp]),
    "cnhip_graph_begin_capture": (i32, [vp]),
    "cnhip_graph_end_capture": (i32, [vp, i32, C.POINTER(vp)]),
    "cnhip_graph_launch": (i32, [vp, vp]),
    "cnhip_graph_destroy": (i32, [vp]),
    "cnhip_gemm_f32": (i32, [i32, i32, i64, i64, i64, f32, vp, i64, vp, i64, f32, vp, i64, vp,
                             i32, vp]),
    "cnhip_gemm_f32_batched": (i32, [i32, i32, i64, i64, i64, f32, vp, i64, i64, vp, i64, i64,
                                     f32, vp, i64, i64, i64, vp]),
    "cnhip_gemm_timing_enable": (i32, [i32]),
    "cnhip_gemm_timing_read": (i32, [C.POINTER(i64), C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    "cnhip_hbm_timing_enable": (i32, [i32]),
    "cnhip_hbm_timing_read": (i32, [C.c_void_p, i32, C.POINTER(i32)]),
    "cnhip_linear_forward": (i32, [vp, vp, vp, vp, i64, i64, i64, vp]),
    "cnhip_linear_backward": (i32, [vp, vp, vp, vp, vp, vp, i64, i64, i64, i32, i32, vp]),
    "cnhip_column_sum": (i32, [vp, vp, i64, i64, i32, vp]),
    "cnhip_linear_forward_act": (i32, [vp, vp, vp, vp, vp, i64, i64, i64, i32, vp]),
    "cnhip_linear_backward_act": (i32, [vp] * 7 + [i64, i64, i64, i32, i32, i32, vp]),
    "cnhip_linear_backward_act_noalloc": (i32, [vp] * 7 + [i64, i64, i64, i32, i32, i32, vp]),
    "cnhip_conv2d_forward": (i32, [vp, vp, vp, vp] + [i64] * 8 + [vp]),
    "cnhip_conv2d_forward_relu": (i32, [vp, vp, vp, vp] + [i64] * 8 + [vp]),
    "cnhip_conv2d_forward_relu_maxpool": (i32, [vp, vp, vp, vp, vp] + [i64] * 10 + [vp]),
    "cnhip_conv2d_backward": (i32, [vp, vp, vp, vp, vp, vp] + [i64] * 8 + [vp]),
    "cnhip_conv2d_backward_maxpool_relu": (i32, [vp] * 6 + [i64] * 10 + [vp]),
    "cnhip_conv2d_backward_maxpool_relu_fits": (i32, [i64] * 10),
    "cnhip_maxpool2d_forward": (i32, [vp, vp, vp] + [i64] * 6 + [vp]),
    "cnhip_maxpool2d_backward": (i32, [vp, vp, vp] + [i64] * 6 + [vp]),
    "cnhip_maxpool2d_backward_relu": (i32, [vp, vp, vp, vp] + [i64] * 6 + [vp]),
    "cnhip_maxpool2d_backward_relu_pooled": (i32, [vp, vp, vp, vp] + [i64] * 6 + [vp]),
    "cnhip_linear_backward_maxpool_relu": (i32, [vp] * 7 + [i64] * 7 + [i32, vp]),
    "cnhip_linear_backward_maxpool_relu_fits": (i32, [i64] * 7),
    "cnhip_recurrence_fault_check": (i32, [vp]),
    "cnhip_lstm_phase_stamps": (i32, [vp, vp, i64]),
    "cnhip_update_seq_last": (i64, []),
    "cnhip_update_faults_taken": (i64, []),
    "cnhip_update_withheld": (i32, [i64]),
    "cnhip_lstm_forward": (i32, [vp] * 8 + [i64] * 4 + [vp]),
    "cnhip_lstm_backward": (i32, [vp] * 12 + [i64] * 4 + [vp]),
    "cnhip_lstm_backward_last": (i32, [vp] * 12 + [i64] * 4 + [vp]),
    "cnhip_gru_forward": (i32, [vp] * 7 + [i64] * 4 + [vp]),
    "cnhip_gru_backward": (i32, [vp] * 11 + [i64] * 4 + [vp]),
    "cnhip_seq_select": (i32, [vp, vp, i64, i64, i64, i64, vp]),
    "cnhip_seq_scatter": (i32, [vp, vp, i64, i64, i64, i64, vp]),
    "cnhip_transpose": (i32, [vp, vp, i64, i64, vp]),
    "cnhip_gather_rows": (i32, [vp, vp, vp, i64, i64, i64, vp]),
    "cnhip_gather_batch": (i32, [vp, vp, vp, vp, vp, i64, i64, i64, i64, vp]),
    "cnhip_mha_cache_floats": (i64, [i64, i64, i64]),
    "cnhip_mha_forward": (i32, [vp] * 9 + [i64] * 4 + [vp]),
    "cnhip_mha_backward": (i32, [vp] * 14 + [i64] * 4 + [vp]),
    "cnhip_mha_forward_residual": (i32, [vp] * 10 + [i64] * 4 + [vp]),
    "cnhip_mha_backward_residual": (i32, [vp] * 15 + [i64] * 4 + [vp]),
    "cnhip_embedding_forward": (i32, [vp, vp, vp, i64, i64, i64, i64, vp, vp]),
    "cnhip_embedding_backward": (i32, [vp, vp, vp, i64, i64, i64, i64, vp]),
    "cnhip_mha_forward_rows": (i32, [vp] * 10 + [i64] * 4 + [i32, vp]),
    "cnhip_mha_backward_rows": (i32, [vp] * 15 + [i64] * 4 + [i32, vp]),
    "cnhip_embedding_forward_rows": (i32, [vp, vp, vp, i64, i64, i64, i64, vp, i32, vp]),
    "cnhip_embedding_backward_rows": (i32, [vp, vp, vp, i64, i64, i64, i64, i32, vp]),
    "cnhip_meanpool1d_forward_rows": (i32, [vp, vp, i64, i64, i64, i32, vp]),
    "cnhip_meanpool1d_backward_rows": (i32, [vp, vp, i64, i64, i64, i32, vp]),
    "cnhip_batchnorm_forward": (i32, [vp] * 9 + [i64, i64, f32, f32, vp]),
    "cnhip_batchnorm_forward_eval": (i32, [vp] * 7 + [i64, i64, f32, vp]),
    "cnhip_batchnorm_backward": (i32, [vp] * 9 + [i64, i64, f32, vp]),
    "cnhip_gelu_forward": (i32, [vp, vp, i64, vp]),
    "cnhip_gelu_backward": (i32, [vp, vp, vp, i64, vp]),
    "cnhip_meanpool1d_forward": (i32, [vp, vp, i64, i64, i64, vp]),
    "cnhip_meanpool1d_backward": (i32, [vp, vp, i64, i64, i64, vp]),
    "cnhip_add": (i32, [vp, vp, vp, i64, vp]),
    "cnhip_relu_forward": (i32, [vp, vp, i64, vp]),
    "cnhip_relu_backward": (i32, [vp, vp, vp, i64, vp]),
    "cnhip_sigmoid_forward": (i32, [vp, vp, i64, vp]),
    "cnhip_sigmoid_backward": (i32, [vp, vp, vp, i64, vp]),
    "cnhip_tanh_forward": (i32, [vp, vp, i64, vp]),
    "cnhip_tanh_backward": (i32, [vp, vp, vp, i64, vp]),
    "cnhip_bce_forward": (i32, [vp, vp, vp, i64, i32, vp]),
    "cnhip_softmax_ce_head": (i32, [vp, vp, vp, vp, vp, i64, i64, i32, vp]),
    "cnhip_sigmoid_bce_head": (i32, [vp, vp, vp, vp, vp, i64, i32, i32, vp]),
    "cnhip_bce_backward": (i32, [vp, vp, vp, i64, i32, vp]),
    "cnhip_mse_forward": (i32, [vp, vp, vp, i64, i32, vp]),
    "cnhip_mse_backward": (i32, [vp, vp, vp, i64, i32, vp]),
    "cnhip_mse_head": (i32, [vp, vp, vp, vp, i64, i32, i32, vp]),
    "cnhip_softmax_ce_forward": (i32, [vp, vp, vp, vp, i64, i64, i32, vp]),
    "cnhip_softmax_ce_backward": (i32, [vp, vp, vp, i64, i64, i32, vp]),
    "cnhip_adam_step": (i32, [vp, vp, vp, vp, i64, f32, f32, f32, f32, f32, f32, vp]),
    "cnhip_mlp2_bce_adam_step": (i32, [vp, vp, i64, i64, i64, vp, vp, vp, vp, vp, vp, vp, vp,
                                       C.POINTER(vp), C.POINTER(vp), C.POINTER(f32), C.POINTER(f32),
                                       f32, f32, f32, f32, i32, i32, vp, vp]),
    "cnhip_adam_step_multi": (i32, [i32, C.POINTER(vp), C.POINTER(vp), C.POINTER(vp),
                                    C.POINTER(vp), C.POINTER(i64), C.POINTER(f32),
                                    C.POINTER(f32), f32, f32, f32, f32, vp]),
    "cnhip_optimizer_step_multi": (i32, [i32, i32, C.POINTER(vp), C.POINTER(vp), C.POINTER(vp),
                                         C.POINTER(i64), f32, f32, f32, vp]),
    "cnhip_leaky_relu_forward": (i32, [vp, vp, i64, f32, vp]),
    "cnhip_leaky_relu_backward": (i32, [vp, vp, vp, i64, f32, vp]),
    "cnhip_softmax_forward": (i32, [vp, vp, i64, i64, vp]),
    "cnhip_softmax_backward": (i32, [vp, vp, vp, i64, i64, vp]),
    "cnhip_cce_forward": (i32, [vp, vp, vp, vp, vp, i64, i64, i32, f32, i32, vp]),
    "cnhip_cce_backward": (i32, [vp, vp, vp, i64, i64, i32, i32, vp]),
    "cnhip_mae_forward": (i32, [vp, vp, vp, i64, i32, vp]),
    "cnhip_mae_backward": (i32, [vp, vp, vp, i64, i32, vp]),
    "cnhip_huber_forward": (i32, [vp, vp, vp, i64, f32, i32, vp]),
    "cnhip_huber_backward": (i32, [vp, vp, vp, i64, f32, i32, vp]),
    "cnhip_dropout_forward": (i32, [vp, vp, vp, i64, f32, C.c_uint64, C.c_uint64, vp]),
    "cnhip_dropout_backward": (i32, [vp, vp, vp, i64, f32, vp]),
    "cnhip_global_avgpool_forward": (i32, [vp, vp, i64, i64, i64, i64, vp]),
    "cnhip_global_avgpool_backward": (i32, [vp, vp, i64, i64, i64, i64, vp]),
    "cnhip_global_maxpool_forward": (i32, [vp, vp, vp, vp, i64, i64, i64, i64, vp]),
    "cnhip_global_maxpool_backward": (i32, [vp, vp, vp, vp, i64, i64, i64, i64, vp]),
    "cnhip_rnn_forward": (i32, [vp] * 5 + [i64] * 4 + [vp]),
    "cnhip_rnn_backward": (i32, [vp] * 9 + [i64] * 4 + [vp]),
}


class KernelTiming(C.Structure):
    """cnhip_kernel_timing (include/cnhip.h)."""
    _fields_ = [("kernel", C.c_char_p), ("launches", C.c_int64), ("total_ms", C.c_double),
                ("total_bytes", C.c_double)]


def hbm_timing_rows() -> list[dict]:
    """Rows of cnhip_hbm_timing_read as dicts (kernel, launches, total_ms, total_bytes)."""
    lib = load()
    n = C.c_int()
    check(lib.cnhip_hbm_timing_read(None, 0, C.byref(n)))
    rows = (KernelTiming * max(1, n.value))()
    check(lib.cnhip_hbm_timing_read(C.cast(rows, C.c_void_p), n.value, C.byref(n)))
    return [{"kernel": r.kernel.decode(), "launches": r.launches, "total_ms": r.total_ms,
             "total_bytes": r.total_bytes} for r in rows[:n.value]]


class CnhipError(RuntimeError):
    """Non-zero status from the HIP library; the message is cnhip_last_error()."""


_lib = None


def header_symbols(header: Path = HEADER) -> list[str]:
    """Function names declared in a C header (used by the export test)."""
    text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(cn[a-z]*_[a-z0-9_]+)\s*\(", text)))


def lib_path() -> Path:
    return LIBDIR / "libcnhip.so"


def load() -> C.CDLL:
    """Load libcnhip.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    path = lib_path()
    if not path.exists():
        raise ImportError(f"{path} is missing: run `python -m cppnet_amd.build` first "
                          "(there is no CPU fallback)")
    lib = C.CDLL(str(path), mode=C.RTLD_GLOBAL)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(status: int) -> None:
    if status != 0:
        msg = load().cnhip_last_error().decode(errors="replace")
        raise CnhipError(f"cnhip status {status}: {msg}")


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args))
