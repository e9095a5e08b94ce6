"""CPU oracle (TEST INFRASTRUCTURE ONLY): ctypes binding of oracle/liboracle.so.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and
only as the checker or the timed CPU baseline. It restates the reference's CPU path (see
oracle/le_oracle.c for the file:line of each function) and is never called by lastengine_amd.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    path = os.path.join(HERE, "liboracle.so")
    if not os.path.exists(path):
        subprocess.run(["make", "-s", "-C", HERE], check=True)
    L = ctypes.CDLL(path)
    P, I, S, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_float
    sig = {
        "or_f16_to_f32": (F, [ctypes.c_uint16]),
        "or_ksign": (ctypes.c_uint8, [I]),
        "or_row_bytes": (S, [I, S]),
        "or_dequant_rows": (I, [I, P, P, S, S]),
        "or_matmat": (I, [I, P, S, S, P, S, P, I]),
        "or_matvec": (I, [I, P, S, S, P, P, I]),
        "or_route": (None, [P, I, I, P, P]),
        "or_moe": (I, [I, I, I, P, P, P, I, I, S, S, P, P, I, P, P, P, I]),
        "or_quant_x": (None, [P, P, P, P, S]),
        "or_matvec_q8": (I, [I, P, S, S, P, P, P, P]),
        "or_rms": (None, [P, P, P, S, F]),
        "or_swiglu": (None, [P, P, P, S]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _threads(n):
    return n if n else max(1, min(16, os.cpu_count() or 1))


def f16_to_f32(h):
    return lib().or_f16_to_f32(int(h))


def ksign(i):
    return int(lib().or_ksign(int(i)))


def row_bytes(ty, n):
    return int(lib().or_row_bytes(ty, n))


def dequant_rows(ty, w, rows, cols):
    """quant::dequant_row over `rows` rows (src/quant.rs:59-170) -> float32 (rows, cols)."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    assert w.size >= rows * row_bytes(ty, cols)
    out = np.empty((rows, cols), dtype=np.float32)
    if not lib().or_dequant_rows(ty, w.ctypes.data, out.ctypes.data, rows, cols):
        raise ValueError("unsupported type %d" % ty)
    return out


def matmat(ty, w, rows, cols, x, nthreads=0):
    """cpu_ref::matmat (src/cpu_ref.rs:266-276): x (m, cols) -> (m, rows)."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    m = x.shape[0]
    assert x.shape[1] == cols
    y = np.empty((m, rows), dtype=np.float32)
    if not lib().or_matmat(ty, w.ctypes.data, rows, cols, x.ctypes.data, m, y.ctypes.data, _threads(nthreads)):
        raise ValueError("unsupported type %d" % ty)
    return y


def matvec(ty, w, rows, cols, x, nthreads=0):
    """cpu_ref::matvec (src/cpu_ref.rs:109-118) -> (rows,)."""
    return matmat(ty, w, rows, cols, np.asarray(x, dtype=np.float32).reshape(1, cols), nthreads)[0]


def route(logits, k):
    """Routing of cpu_ref::moe (src/cpu_ref.rs:243-250) -> (idx[k], w[k])."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    idx = np.empty(k, dtype=np.int32)
    w = np.empty(k, dtype=np.float32)
    lib().or_route(lg.ctypes.data, lg.size, k, idx.ctypes.data, w.ctypes.data)
    return idx, w


def moe(ty_g, ty_u, ty_d, gate, up, down, n_exp, k, hidden, ff, h, logits, nthreads=0):
    """Routed part of cpu_ref::moe (src/cpu_ref.rs:242-259) for n_tok tokens.
    Returns (out (n_tok, hidden), idx (n_tok, k), w (n_tok, k))."""
    h = np.ascontiguousarray(np.atleast_2d(h), dtype=np.float32)
    lg = np.ascontiguousarray(np.atleast_2d(logits), dtype=np.float32)
    n_tok = h.shape[0]
    out = np.empty((n_tok, hidden), dtype=np.float32)
    idx = np.empty((n_tok, k), dtype=np.int32)
    w = np.empty((n_tok, k), dtype=np.float32)
    g, u, d = (np.ascontiguousarray(a, dtype=np.uint8) for a in (gate, up, down))
    ok = lib().or_moe(ty_g, ty_u, ty_d, g.ctypes.data, u.ctypes.data, d.ctypes.data, n_exp, k, hidden, ff,
                      h.ctypes.data, lg.ctypes.data, n_tok, out.ctypes.data, idx.ctypes.data, w.ctypes.data,
                      _threads(nthreads))
    if not ok:
        raise ValueError("bad moe arguments")
    return out, idx, w


def quant_x(x):
    """quant_x (src/cuda/kernels.cu:15-25) over a length-32n vector -> (xq int8, xd f32, xs i32)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    assert x.size % 32 == 0
    n = x.size // 32
    xq = np.empty(x.size, dtype=np.int8)
    xd = np.empty(n, dtype=np.float32)
    xs = np.empty(n, dtype=np.int32)
    lib().or_quant_x(x.ctypes.data, xq.ctypes.data, xd.ctypes.data, xs.ctypes.data, n)
    return xq, xd, xs


def matvec_q8(ty, w, rows, cols, xq, xd, xs):
    """matvec_<ty> on int8 activations (src/cuda/kernels.cu:36-110,371-392) -> (rows,)."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    xd = np.ascontiguousarray(xd, dtype=np.float32)
    xs = np.ascontiguousarray(xs, dtype=np.int32)
    y = np.empty(rows, dtype=np.float32)
    if not lib().or_matvec_q8(ty, w.ctypes.data, rows, cols, xq.ctypes.data, xd.ctypes.data, xs.ctypes.data, y.ctypes.data):
        raise ValueError("unsupported type %d or shape" % ty)
    return y


def rms(x, w, eps):
    """cpu_ref::rms (src/cpu_ref.rs:32-36): x * (1 / sqrt(mean(x^2) + eps)) * w."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    o = np.empty_like(x)
    lib().or_rms(x.ctypes.data, w.ctypes.data, o.ctypes.data, x.size, float(eps))
    return o


def swiglu(g, u):
    """silu(g) * u as cpu_ref computes it (src/cpu_ref.rs:37,255)."""
    g = np.ascontiguousarray(g, dtype=np.float32).reshape(-1)
    u = np.ascontiguousarray(u, dtype=np.float32).reshape(-1)
    o = np.empty_like(g)
    lib().or_swiglu(g.ctypes.data, u.ctypes.data, o.ctypes.data, g.size)
    return o
