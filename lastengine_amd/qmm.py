"""ctypes binding of lible_qmm.so (include/le_qmm.h, include/le_quant.h).

`Engine` mirrors the reference's launch surface for this path (src/gpu.rs:223-238 `mv_ptrs`/`mv`,
src/gpu/prefill.rs:44-60 `mm`/`dense`, src/gpu/dense.rs:181-199 `bmm`): a context over the loaded
gfx950 code objects whose methods take device buffers and launch on the current stream. Errors
come back as LeError carrying the C status code (the reference panics on the same conditions,
src/gpu.rs:221,233).

Device buffers may be passed as torch tensors (their data_ptr is used) or as raw integer
addresses. There is no CPU fallback: without the built library or a gfx950 device every entry
raises.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(HERE, "lib")

Q4_0, Q8_0, Q3_K, Q4_K, Q5_K, Q6_K, IQ2_XXS, IQ3_XXS, IQ2_S = 2, 8, 11, 12, 13, 14, 16, 18, 22
# the five types of every entry point (and of this build's quantizer)
TYPES = {"Q8_0": Q8_0, "Q4_K": Q4_K, "Q6_K": Q6_K, "IQ2_XXS": IQ2_XXS, "IQ3_XXS": IQ3_XXS}
# types that le_dequant_rows, le_matvec, le_matvec_q8 and le_gemm also accept
MV_TYPES = dict(TYPES, Q4_0=Q4_0, Q3_K=Q3_K, Q5_K=Q5_K, IQ2_S=IQ2_S)
# (gate/up, down) type pairs of the decode-shaped MoE kernels; every other pair of MV_TYPES runs the
# grouped form, whose workspace is le_moe_prefill_workspace_size at any token count
MOE_DECODE_PAIRS = {(Q4_K, Q6_K), (Q4_K, Q4_K), (Q6_K, Q6_K), (Q8_0, Q8_0), (IQ2_XXS, IQ3_XXS), (IQ2_XXS, IQ2_XXS),
                    (IQ3_XXS, IQ3_XXS)}

_STATUS = {0: "ok", -1: "invalid argument", -2: "unsupported quant type", -3: "unsupported shape",
           -4: "misaligned pointer or stride", -5: "HIP runtime error",
           -6: "code object missing or device unsupported", -7: "workspace too small",
           -8: "a bounded device-side wait gave up"}


class LeError(RuntimeError):
    def __init__(self, code, msg=""):
        self.code = code
        super().__init__("le_qmm error %d (%s)%s" % (code, _STATUS.get(code, "?"), (": " + msg) if msg else ""))


def library_path():
    return os.path.join(LIB_DIR, "lible_qmm.so")


_lib = None


def lib():
    """Load lible_qmm.so once and declare the C signatures."""
    global _lib
    if _lib is not None:
        return _lib
    path = library_path()
    if not os.path.exists(path):
        raise LeError(-6, "%s is not built; run __graft_entry__.build() or lastengine_amd/build.py" % path)
    L = ctypes.CDLL(path)
    P, I, LL, S, F, D = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_size_t, ctypes.c_float, ctypes.c_double
    sig = {
        "le_block_info": (I, [I, ctypes.POINTER(I), ctypes.POINTER(I)]),
        "le_row_bytes": (S, [I, S]),
        "le_status_str": (ctypes.c_char_p, [I]),
        "le_init": (I, [ctypes.c_char_p, ctypes.POINTER(P)]),
        "le_destroy": (None, [P]),
        "le_last_error": (ctypes.c_char_p, [P]),
        "le_set_option": (I, [P, ctypes.c_char_p, I]),
        "le_dequant_rows": (I, [P, I, P, P, I, I, P]),
        "le_matvec": (I, [P, I, P, P, P, LL, P, I, I, I, P]),
        "le_quant_x": (I, [P, P, P, P, P, I, P]),
        "le_matvec_swiglu": (I, [P, I, P, P, P, LL, P, I, I, I, P]),
        "le_rms_quant": (I, [P, P, P, P, P, P, P, I, F, P]),
        "le_matvec_q8": (I, [P, I, P, P, P, P, P, LL, P, I, I, I, P]),
        "le_gemm_workspace_size": (S, [I, I, I]),
        "le_gemm_workspace_size_rows": (S, [I, I, I, I]),
        "le_gemm": (I, [P, I, P, P, I, P, I, I, P, S, P]),
        "le_gemm_noalloc": (I, [P, I, P, P, I, P, I, I, P]),
        "le_stream_read": (I, [P, P, S, P, P]),
        "le_stream_read_sink_bytes": (I, [P]),
        "le_moe_workspace_size": (S, [I, I, I]),
        "le_moe_layer": (I, [P, I, I, I, P, P, P, I, I, I, I, P, P, I, P, P, P, P, S, P]),
        "le_moe_check": (I, [P, P, P]),
        "le_moe_prefill_workspace_size": (S, [I, I, I, I, I]),
        "le_moe_layer_ptrs": (I, [P, I, I, I, P, P, P, I, I, I, I, P, P, I, P, P, P, P, S, P]),
        "le_mm_grouped_workspace_size": (S, [I, I, I, I]),
        "le_mm_grouped": (I, [P, I, P, P, P, P, P, I, I, P, P, I, I, P, S, P]),
        "le_fill_normal": (None, [P, S, ctypes.c_uint64, ctypes.c_uint64, D, D, I]),
        "le_quantize_rows": (I, [I, P, P, S, S, I]),
        "le_f32_to_f16": (ctypes.c_uint16, [F]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _threads():
    return max(1, min(16, os.cpu_count() or 1))


def block_info(ty):
    v, b = ctypes.c_int(), ctypes.c_int()
    rc = lib().le_block_info(ty, ctypes.byref(v), ctypes.byref(b))
    if rc:
        raise LeError(rc)
    return v.value, b.value


def row_bytes(ty, n):
    return int(lib().le_row_bytes(ty, n))


def f32_to_f16(x):
    return int(lib().le_f32_to_f16(float(x)))


def fill_normal(n, seed, std=1.0, mean=0.0, offset=0):
    """Seeded N(mean, std) float32 vector (splitmix64 + Box-Muller, see include/le_quant.h)."""
    out = np.empty(int(n), dtype=np.float32)
    lib().le_fill_normal(out.ctypes.data, out.size, ctypes.c_uint64(seed), ctypes.c_uint64(offset),
                         float(mean), float(std), _threads())
    return out


def quantize_rows(ty, x):
    """Quantize a (rows, cols) float32 array into GGUF blocks -> uint8 array (rows, row_bytes)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    out = np.empty((rows, row_bytes(ty, cols)), dtype=np.uint8)
    rc = lib().le_quantize_rows(ty, x.ctypes.data, out.ctypes.data, rows, cols, _threads())
    if rc:
        raise LeError(rc)
    return out


def _ptr(t):
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(stream):
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


class Engine:
    """One le_ctx: the gfx950 code objects loaded on the current device."""

    def __init__(self, lib_dir=None):
        import torch  # torch must bring up its HIP context before this library touches the runtime
        if torch.cuda.is_available():
            torch.cuda.init()
        self._L = lib()
        self._ctx = ctypes.c_void_p()
        rc = self._L.le_init(lib_dir.encode() if lib_dir else None, ctypes.byref(self._ctx))
        if rc:
            raise LeError(rc, "le_init (needs a gfx950 device and the built code objects in %s)" % (lib_dir or LIB_DIR))

    def close(self):
        if self._ctx:
            self._L.le_destroy(self._ctx)
            self._ctx = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc):
        if rc:
            raise LeError(rc, (self._L.le_last_error(self._ctx) or b"").decode())

    def set_option(self, name, value):
        self._check(self._L.le_set_option(self._ctx, name.encode(), int(value)))

    def dequant_rows(self, ty, w, out, rows, cols, stream=None):
        self._check(self._L.le_dequant_rows(self._ctx, ty, _ptr(w), _ptr(out), rows, cols, _stream(stream)))

    def mv_ptrs(self, ty, ptrs, x, out, rows, cols, xstride, slots, w=None, stream=None):
        """Gpu::mv_ptrs (src/gpu.rs:228): out[s*rows + r] = W_s[r] . x[s*xstride:]."""
        self._check(self._L.le_matvec(self._ctx, ty, _ptr(ptrs), _ptr(w), _ptr(x), int(xstride), _ptr(out), rows,
                                      cols, slots, _stream(stream)))

    def mv_swiglu(self, ty, w, gu, out, rows, cols, ptrs=None, xstride=0, slots=1, stream=None):
        """swiglu_gu + down matvec in one launch: out = W . (silu(gu[:cols]) * gu[cols:2 cols])."""
        self._check(self._L.le_matvec_swiglu(self._ctx, ty, _ptr(ptrs), _ptr(w), _ptr(gu), int(xstride), _ptr(out), rows,
                                             cols, slots, _stream(stream)))

    def quant_x(self, x, xq, xd, xs, n_units, stream=None):
        """Gpu::qx / quant_x (src/gpu.rs:223, src/cuda/kernels.cu:15-25): int8 activations per 32 values."""
        self._check(self._L.le_quant_x(self._ctx, _ptr(x), _ptr(xq), _ptr(xd), _ptr(xs), int(n_units), _stream(stream)))

    def rms_quant(self, x, w, o, xq, xd, xs, n, eps, stream=None):
        """rms_quant (src/cuda/dense.cu:33-56): RMSNorm into o and its int8 quantization."""
        self._check(self._L.le_rms_quant(self._ctx, _ptr(x), _ptr(w), _ptr(o), _ptr(xq), _ptr(xd), _ptr(xs), int(n),
                                         float(eps), _stream(stream)))

    def mv_q8(self, ty, ptrs, xq, xd, xs, out, rows, cols, xstride, slots, w=None, stream=None):
        """matvec_<ty> on quantized activations (src/cuda/kernels.cu:371-392) through le_matvec_q8."""
        self._check(self._L.le_matvec_q8(self._ctx, ty, _ptr(ptrs), _ptr(w), _ptr(xq), _ptr(xd), _ptr(xs), int(xstride),
                                         _ptr(out), rows, cols, slots, _stream(stream)))

    def mv(self, ty, w, x, out, rows, cols, stream=None):
        """Gpu::mv (src/gpu.rs:238): one matrix, one activation."""
        self.mv_ptrs(ty, None, x, out, rows, cols, 0, 1, w=w, stream=stream)

    def moe_workspace_size(self, n_tok, k, ff):
        return int(self._L.le_moe_workspace_size(n_tok, k, ff))

    def moe_prefill_workspace_size(self, n_tok, k, n_exp, hidden, ff):
        return int(self._L.le_moe_prefill_workspace_size(n_tok, k, n_exp, hidden, ff))

    def moe(self, ty_gate, ty_up, ty_down, gate, up, down, n_exp, k, hidden, ff, logits, h, n_tok, out,
            idx_out=None, w_out=None, ws=None, ws_bytes=None, stream=None):
        """Routed MoE layer (cpu_ref::moe, src/cpu_ref.rs:242-259) for n_tok tokens."""
        if ws is None:
            import torch
            n = self.moe_workspace_size(n_tok, k, ff)
            if n_tok >= 11 or (ty_gate, ty_down) not in MOE_DECODE_PAIRS:
                n = max(n, self.moe_prefill_workspace_size(n_tok, k, n_exp, hidden, ff))
            ws = torch.zeros(max(16, n), dtype=torch.uint8, device="cuda")
        if ws_bytes is None:
            ws_bytes = ws.numel() if hasattr(ws, "numel") else 0
        self._check(self._L.le_moe_layer(self._ctx, ty_gate, ty_up, ty_down, _ptr(gate), _ptr(up), _ptr(down), n_exp,
                                         k, hidden, ff, _ptr(logits), _ptr(h), n_tok, _ptr(out), _ptr(idx_out),
                                         _ptr(w_out), _ptr(ws), ws_bytes, _stream(stream)))

    def moe_ptrs(self, ty_gate, ty_up, ty_down, gate_ptrs, up_ptrs, down_ptrs, n_exp, k, hidden, ff, logits, h, n_tok,
                 out, idx_out=None, w_out=None, ws=None, ws_bytes=None, stream=None):
        """The MoE layer over per-expert pointer tables (device arrays of n_exp weight pointers)."""
        if ws is None:
            import torch
            n = self.moe_workspace_size(n_tok, k, ff)
            if n_tok >= 11 or (ty_gate, ty_down) not in MOE_DECODE_PAIRS:
                n = max(n, self.moe_prefill_workspace_size(n_tok, k, n_exp, hidden, ff))
            ws = torch.zeros(max(16, n), dtype=torch.uint8, device="cuda")
        if ws_bytes is None:
            ws_bytes = ws.numel() if hasattr(ws, "numel") else 0
        self._check(self._L.le_moe_layer_ptrs(self._ctx, ty_gate, ty_up, ty_down, _ptr(gate_ptrs), _ptr(up_ptrs),
                                              _ptr(down_ptrs), n_exp, k, hidden, ff, _ptr(logits), _ptr(h), n_tok,
                                              _ptr(out), _ptr(idx_out), _ptr(w_out), _ptr(ws), ws_bytes, _stream(stream)))

    def mm_grouped_workspace_size(self, ty, nslot, npair, cols):
        return int(self._L.le_mm_grouped_workspace_size(ty, nslot, npair, cols))

    def mm_grouped(self, ty, off, in_idx, out_idx, nslot, npair, x, y, rows, cols, ptrs=None, w=None, ws=None,
                   ws_bytes=None, stream=None):
        """prefill::mm / mm_impl (src/cuda/kernels.cu:679-719): y[out_idx[i]] = W_s . x[in_idx[i]] for the
        pairs i of slot s (off[s] .. off[s+1])."""
        if ws is None:
            import torch
            ws = torch.empty(max(16, self.mm_grouped_workspace_size(ty, nslot, npair, cols)), dtype=torch.uint8,
                             device="cuda")
        if ws_bytes is None:
            ws_bytes = ws.numel() if hasattr(ws, "numel") else 0
        self._check(self._L.le_mm_grouped(self._ctx, ty, _ptr(ptrs), _ptr(w), _ptr(off), _ptr(in_idx), _ptr(out_idx),
                                          nslot, npair, _ptr(x), _ptr(y), rows, cols, _ptr(ws), ws_bytes,
                                          _stream(stream)))

    def moe_check(self, ws, stream=None):
        """Raise LeError(-8) if a one-launch MoE layer on workspace ws gave up at its device-wide
        barrier since the last check (synchronizes the stream)."""
        self._check(self._L.le_moe_check(self._ctx, _ptr(ws), _stream(stream)))

    def gemm_workspace_size(self, ty, m, cols):
        return int(self._L.le_gemm_workspace_size(ty, m, cols))

    def gemm_workspace_size_rows(self, ty, m, rows, cols):
        """Workspace that also holds the K slices' partial results (reproducible sums)."""
        return int(self._L.le_gemm_workspace_size_rows(ty, m, rows, cols))

    def gemm(self, ty, w, x, m, out, rows, cols, ws=None, ws_bytes=None, stream=None):
        """DenseGpu::bmm (src/gpu/dense.rs:181): out[t*rows + r] = W[r] . x[t] for t < m."""
        if ws is None:
            n = self.gemm_workspace_size_rows(ty, m, rows, cols)
            if n:
                import torch
                ws = torch.empty(n, dtype=torch.uint8, device="cuda")
        if ws_bytes is None:
            ws_bytes = ws.numel() if hasattr(ws, "numel") else 0
        self._check(self._L.le_gemm(self._ctx, ty, _ptr(w), _ptr(x), m, _ptr(out), rows, cols, _ptr(ws), ws_bytes,
                                    _stream(stream)))

    def gemm_noalloc(self, ty, w, x, m, out, rows, cols, stream=None):
        """le_gemm with the library's per-GPU scratch array as workspace: allocates nothing
        (for graph capture and serving loops). Calls overlapping on one GPU race."""
        self._check(self._L.le_gemm_noalloc(self._ctx, ty, _ptr(w), _ptr(x), m, _ptr(out), rows, cols,
                                            _stream(stream)))

    def stream_read(self, buf, nbytes, sink, stream=None):
        """Streaming-read probe over nbytes of buf (the practical HBM read ceiling at that size)."""
        self._check(self._L.le_stream_read(self._ctx, _ptr(buf), int(nbytes), _ptr(sink), _stream(stream)))

    def stream_read_sink_bytes(self):
        return int(self._L.le_stream_read_sink_bytes(self._ctx))
