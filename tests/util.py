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


def wbytes(ty, rows, cols, seed):
    """Weight bytes for a type: seeded N(0, 0.02) weights through the product quantizer where it has
    one (the five config types), else arbitrary block bytes with bounded finite scales."""
    if ty in le.TYPES.values():
        return weights(ty, rows, cols, seed)[0]
    return random_blocks(ty, rows, cols, seed)


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


# Byte offsets of the f16 scale fields in each block: (block bytes, [field offsets]).
SCALE_FIELDS = {8: (34, [0]), 12: (144, [0, 2]), 14: (210, [208]), 16: (66, [0]), 18: (98, [0]),
                2: (18, [0]), 11: (110, [108]), 13: (176, [0, 2]), 22: (82, [0])}


def random_blocks(ty, rows, cols, seed, dmax=0.01):
    """Arbitrary GGUF block bytes (every scale/min code, grid index, sign pattern and, for Q6_K,
    negative sub-block scales) with the f16 super-block scale fields replaced by finite values
    drawn uniformly from [-dmax, dmax], as real GGUF tensors have."""
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 256, size=(rows, le.row_bytes(ty, cols)), dtype=np.uint8)
    bb, offs = SCALE_FIELDS[ty]
    nblk = q.shape[1] // bb
    blk = q.reshape(rows, nblk, bb)
    for o in offs:
        d = rng.uniform(-dmax, dmax, size=(rows, nblk)).astype(np.float16)
        blk[:, :, o:o + 2] = d.view(np.uint8).reshape(rows, nblk, 2)
    return q
