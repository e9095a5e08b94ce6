"""Shared helpers for the parity tests (seeded inputs, tolerance checks)."""
import numpy as np

import lastengine_amd as le

# Parity bar for dot/GEMM outputs: max|got-want| / max|want| <= 1e-3 and, per output,
# |got-want| <= 1e-3 * sum|w*x| (the condition-aware form of the reference's own GPU test,
# src/gpu.rs:730-731, which uses 0.05 instead of 1e-3).
REL_TOL = 1e-3


def weights(ty, rows, cols, seed, std=0.02):
    """Seeded N(0, std) weights quantized with the product quantizer -> (bytes, fp32 source)."""
    src = le.fill_normal(rows * cols, seed, std=std).reshape(rows, cols)
    return le.quantize_rows(ty, src), src


def acts(n, seed):
    return le.fill_normal(n, seed)


def check_close(got, want, absmag):
    """got/want (..., rows); absmag = sum|w*x| per output (same shape)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    err = np.abs(got - want)
    assert np.all(np.isfinite(got)), "non-finite output"
    mx = float(np.max(np.abs(want))) if want.size else 0.0
    norm_err = float(err.max() / mx) if mx > 0 else float(err.max())
    assert norm_err <= REL_TOL, "max|got-want|/max|want| = %.3e > %.0e" % (norm_err, REL_TOL)
    bound = REL_TOL * np.asarray(absmag, dtype=np.float64) + 1e-30
    worst = float(np.max(err / bound))
    assert worst <= 1.0, "per-output error %.3f x of 1e-3*sum|wx|" % worst
    return norm_err, worst
