"""Test-side access to the CPU oracle (oracle/) plus the tolerance helpers
the parity tests share."""
from __future__ import annotations

import numpy as np

from oracle import ORACLE_SO, colmajor, fp, from_colmajor, load_oracle  # noqa: F401


def close(a, b, rtol=1e-4, atol=1e-5) -> tuple[bool, str]:
    """Elementwise |a-b| <= atol + rtol*|b| (b is the reference)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    if a.shape != b.shape:
        return False, f"shape {a.shape} vs {b.shape}"
    err = np.abs(a - b)
    lim = atol + rtol * np.abs(b)
    bad = err > lim
    if not np.all(np.isfinite(a)):
        return False, "non-finite values"
    if bad.any():
        i = int(np.argmax(err - lim))
        return False, (f"{int(bad.sum())}/{a.size} outside rtol={rtol} atol={atol}; worst at {i}:"
                       f" got {a.flat[i]!r} want {b.flat[i]!r}")
    return True, f"max abs err {err.max() if err.size else 0:.3g}"


def close_mag(a, b, mag, rtol=1e-4, atol=1e-5) -> tuple[bool, str]:
    """Condition-aware fp32 bound for contractions:
    |a-b| <= atol + rtol * max(|b|, mag), where mag = (|A| |B|) / sqrt(K) is
    the RMS size of the partial sums of each dot product.  Elementwise rel
    1e-4 alone cannot hold where a length-K fp32 sum cancels to ~0 (both the
    oracle's and the GPU's rounding are ~u*sqrt(K)*mag there)."""
    b64 = np.abs(np.asarray(b, np.float64))
    m64 = np.asarray(mag, np.float64)
    return _close_lim(a, b, atol + rtol * np.maximum(b64, m64), rtol, atol)


def _close_lim(a, b, lim, rtol, atol):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    if a.shape != b.shape:
        return False, f"shape {a.shape} vs {b.shape}"
    if not np.all(np.isfinite(a)):
        return False, "non-finite values"
    err = np.abs(a - b)
    bad = err > lim
    if bad.any():
        i = int(np.argmax(err - lim))
        return False, (f"{int(bad.sum())}/{a.size} outside rtol={rtol} atol={atol} (magnitude-aware);"
                       f" worst at {i}: got {a.flat[i]!r} want {b.flat[i]!r} lim {lim.flat[i]!r}")
    return True, f"max abs err {err.max() if err.size else 0:.3g}"


def gemm_mag(oracle, ta, tb, M, N, K, A, lda, B, ldb, ldc):
    """(|op(A)| |op(B)|) / sqrt(K) laid out like C (ld = ldc), via the oracle."""
    mag = np.zeros(max(1, ldc * N), np.float32)
    if K > 0:
        oracle.cnref_gemm_f32(ta, tb, M, N, K, 1.0 / float(np.sqrt(K)), fp(np.abs(A)), lda,
                              fp(np.abs(B)), ldb, 0.0, fp(mag), ldc, None, 0)
    return mag[: ldc * N]
