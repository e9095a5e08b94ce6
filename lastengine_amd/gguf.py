"""ctypes binding of the GGUF reader (include/le_gguf.h), mirroring the reference's Gguf
(src/gguf.rs:36-44, open :95-122) and the tensor access of cpu_ref::Model (src/cpu_ref.rs:56-58,
70-85): `version`, `kv` lookups with the reference's as_u64 / as_f32 / as_str meanings, `tensors`
(name, dims, ggml type, absolute offset, bytes), `data_start`, expert slabs of 3D tensors, and
raw tensor bytes ready to upload to the device."""
import ctypes

import numpy as np

from .qmm import LeError, lib

_SIG = False


def _L():
    global _SIG
    L = lib()
    if not _SIG:
        P, I, U64, CP = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64, ctypes.c_char_p
        sig = {
            "le_gguf_open": (I, [CP, ctypes.POINTER(P)]),
            "le_gguf_open_error": (CP, []),
            "le_gguf_close": (None, [P]),
            "le_gguf_version": (I, [P]),
            "le_gguf_data_start": (U64, [P]),
            "le_gguf_tensor_count": (I, [P]),
            "le_gguf_kv_count": (I, [P]),
            "le_gguf_find": (I, [P, CP]),
            "le_gguf_tensor_info": (I, [P, I, ctypes.POINTER(CP), ctypes.POINTER(I), ctypes.POINTER(I),
                                        ctypes.POINTER(U64), ctypes.POINTER(U64), ctypes.POINTER(U64)]),
            "le_gguf_expert_slab": (I, [P, CP, I, ctypes.POINTER(U64), ctypes.POINTER(U64)]),
            "le_gguf_kv_type": (I, [P, CP]),
            "le_gguf_kv_u64": (I, [P, CP, ctypes.POINTER(U64)]),
            "le_gguf_kv_i64": (I, [P, CP, ctypes.POINTER(ctypes.c_int64)]),
            "le_gguf_kv_f32": (I, [P, CP, ctypes.POINTER(ctypes.c_float)]),
            "le_gguf_kv_str": (I, [P, CP, ctypes.POINTER(CP)]),
            "le_gguf_kv_array": (I, [P, CP, ctypes.POINTER(I), ctypes.POINTER(U64)]),
            "le_gguf_read": (I, [P, U64, U64, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _SIG = True
    return L


class TensorInfo:
    __slots__ = ("name", "dims", "ggml_type", "offset", "nbytes", "fits")

    def __init__(self, name, dims, ggml_type, offset, nbytes, fits=True):
        self.name, self.dims, self.ggml_type, self.offset, self.nbytes = name, dims, ggml_type, offset, nbytes
        self.fits = fits

    def __repr__(self):
        return "TensorInfo(%r, dims=%r, type=%d, offset=%d, nbytes=%d)" % (
            self.name, self.dims, self.ggml_type, self.offset, self.nbytes)


class Gguf:
    """Gguf::open (src/gguf.rs:95-122). Raises LeError on a malformed file."""

    def __init__(self, path):
        L = _L()
        self._g = ctypes.c_void_p()
        rc = L.le_gguf_open(str(path).encode(), ctypes.byref(self._g))
        if rc:
            raise LeError(rc, (L.le_gguf_open_error() or b"").decode())
        self.path = str(path)
        self.version = L.le_gguf_version(self._g)
        self.data_start = int(L.le_gguf_data_start(self._g))
        self.tensors = [self._info(i) for i in range(L.le_gguf_tensor_count(self._g))]
        self.kv_count = L.le_gguf_kv_count(self._g)

    def close(self):
        if self._g:
            _L().le_gguf_close(self._g)
            self._g = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _info(self, i):
        name, ty, nd = ctypes.c_char_p(), ctypes.c_int(), ctypes.c_int()
        dims, off, nb = (ctypes.c_uint64 * 8)(), ctypes.c_uint64(), ctypes.c_uint64()
        rc = _L().le_gguf_tensor_info(self._g, i, ctypes.byref(name), ctypes.byref(ty), ctypes.byref(nd), dims,
                                      ctypes.byref(off), ctypes.byref(nb))
        if rc and rc != -3:
            raise LeError(rc)
        t = TensorInfo(name.value.decode(), [int(dims[d]) for d in range(nd.value)], ty.value, off.value, nb.value)
        t.fits = rc == 0  # -3: its size overflows or its data runs past the end of the file
        return t

    def find(self, name):
        i = _L().le_gguf_find(self._g, name.encode())
        return self.tensors[i] if i >= 0 else None

    def kv_type(self, key):
        return _L().le_gguf_kv_type(self._g, key.encode())

    def as_u64(self, key):
        v = ctypes.c_uint64()
        return int(v.value) if _L().le_gguf_kv_u64(self._g, key.encode(), ctypes.byref(v)) == 0 else None

    def as_i64(self, key):
        v = ctypes.c_int64()
        return int(v.value) if _L().le_gguf_kv_i64(self._g, key.encode(), ctypes.byref(v)) == 0 else None

    def as_f32(self, key):
        v = ctypes.c_float()
        return float(v.value) if _L().le_gguf_kv_f32(self._g, key.encode(), ctypes.byref(v)) == 0 else None

    def as_str(self, key):
        v = ctypes.c_char_p()
        return v.value.decode() if _L().le_gguf_kv_str(self._g, key.encode(), ctypes.byref(v)) == 0 else None

    def array(self, key):
        """(element type, length) of an array value, or None."""
        et, n = ctypes.c_int(), ctypes.c_uint64()
        return (et.value, int(n.value)) if _L().le_gguf_kv_array(self._g, key.encode(), ctypes.byref(et),
                                                                 ctypes.byref(n)) == 0 else None

    def arch(self):
        return self.as_str("general.architecture")

    def read(self, offset, nbytes):
        out = np.empty(nbytes, dtype=np.uint8)
        rc = _L().le_gguf_read(self._g, offset, nbytes, out.ctypes.data)
        if rc:
            raise LeError(rc, "read of %d bytes at %d" % (nbytes, offset))
        return out

    def tensor_bytes(self, name):
        t = self.find(name)
        if t is None:
            raise LeError(-1, "missing tensor %s" % name)
        if not t.fits:
            raise LeError(-3, "tensor %s does not fit the file" % name)
        return self.read(t.offset, t.nbytes)

    def expert_slab(self, name, expert):
        """(absolute offset, bytes) of expert `expert` of a 3D tensor (src/cpu_ref.rs:78-85)."""
        off, nb = ctypes.c_uint64(), ctypes.c_uint64()
        rc = _L().le_gguf_expert_slab(self._g, name.encode(), expert, ctypes.byref(off), ctypes.byref(nb))
        if rc:
            raise LeError(rc, "expert %d of %s" % (expert, name))
        return int(off.value), int(nb.value)
