"""Host-side checks of the C ABI that need no GPU: the library loads, exports every function the
headers declare, computes geometry like src/quant.rs:24-35, and rejects bad arguments with status
codes instead of crashing."""
import ctypes
import os
import re

import numpy as np
import pytest

import lastengine_amd as le
from lastengine_amd import qmm
from tests.conftest import REPO

HEADERS = [os.path.join(REPO, "include", h) for h in ("le_qmm.h", "le_quant.h", "le_gguf.h")]


def declared_functions():
    names = []
    for h in HEADERS:
        txt = open(h).read()
        txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\**\s*(le_[a-z_0-9]+)\s*\(", txt, flags=re.M)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    names = declared_functions()
    assert "le_matvec" in names and "le_init" in names and "le_quantize_rows" in names
    L = ctypes.CDLL(qmm.library_path())
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_code_objects_built():
    for part in ("deq", "moe", "gm", "gq", "mv2", "mv8", "mv11", "mv12", "mv13", "mv14", "mv16", "mv18", "mv22"):
        assert os.path.getsize(os.path.join(qmm.LIB_DIR, "le_qmm_%s.hsaco" % part)) > 1000


ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def test_code_objects_use_no_flat_memory_ops(tmp_path):
    """Every kernel addresses global memory and LDS through typed instructions: a flat load or
    store also counts against the LDS wait counter, so each LDS wait in a kernel would wait for
    the weight loads in flight as well (checked on the disassembly of the built code objects)."""
    import subprocess
    bundler = os.path.join(ROCM, "llvm", "bin", "clang-offload-bundler")
    objdump = os.path.join(ROCM, "llvm", "bin", "llvm-objdump")
    if not (os.path.exists(bundler) and os.path.exists(objdump)):
        pytest.skip("ROCm LLVM tools not installed")
    lib = os.path.join(REPO, "lastengine_amd", "lib")
    found = {}
    for name in sorted(os.listdir(lib)):
        if not name.endswith(".hsaco"):
            continue
        elf = str(tmp_path / (name + ".elf"))
        subprocess.run([bundler, "--type=o", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950",
                        "--input=" + os.path.join(lib, name), "--output=" + elf, "--unbundle"], check=True)
        asm = subprocess.run([objdump, "-d", elf], check=True, capture_output=True, text=True).stdout
        n = len(re.findall(r"\bflat_(load|store|atomic)", asm))
        if n:
            found[name] = n
    assert not found, found


@pytest.mark.parametrize("ty,cols,want", [(8, 4096, 4352), (12, 4096, 2304), (14, 14336, 11760),
                                          (16, 4096, 1056), (18, 14336, 5488), (12, 2048, 1152),
                                          (14, 768, 630)])
def test_row_bytes(ty, cols, want):
    assert le.row_bytes(ty, cols) == want


def test_block_info_and_bad_type():
    assert le.block_info(le.Q4_K) == (256, 144)
    assert le.block_info(le.Q8_0) == (32, 34)
    with pytest.raises(le.LeError) as e:
        le.block_info(99)
    assert e.value.code == -2
    assert le.row_bytes(99, 256) == 0


def test_quantize_errors():
    L = qmm.lib()
    x = np.zeros(300, dtype=np.float32)
    out = np.zeros(1024, dtype=np.uint8)
    assert L.le_quantize_rows(12, x.ctypes.data, out.ctypes.data, 1, 300, 1) == -3  # not a block multiple
    assert L.le_quantize_rows(7, x.ctypes.data, out.ctypes.data, 1, 256, 1) == -2
    assert L.le_quantize_rows(12, None, out.ctypes.data, 1, 256, 1) == -1


def test_fill_normal_deterministic_and_threaded():
    a = le.fill_normal(100003, 42)
    L = qmm.lib()
    b = np.empty_like(a)
    L.le_fill_normal(b.ctypes.data, b.size, ctypes.c_uint64(42), ctypes.c_uint64(0), 0.0, 1.0, 1)
    assert np.array_equal(a, b)
    c = le.fill_normal(1000, 42, offset=500)
    assert np.array_equal(c, a[500:1500])
    assert abs(a.mean()) < 0.02 and abs(a.std() - 1) < 0.02


def test_f32_to_f16_matches_numpy():
    rng = np.random.default_rng(5)
    vals = np.concatenate([rng.normal(size=2000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, size=2000),
                           np.array([0.0, -0.0, 65504.0, 65520.0, 1e-8, 5.96e-8, 2.98e-8, np.inf, -np.inf],
                                    dtype=np.float32)])
    for v in vals:
        assert le.f32_to_f16(v) == int(np.array(v, dtype=np.float16).view(np.uint16)), v


def test_quantizer_is_deterministic():
    src = le.fill_normal(4 * 1024, 7, std=0.02).reshape(4, 1024)
    for ty in le.TYPES.values():
        assert np.array_equal(le.quantize_rows(ty, src), le.quantize_rows(ty, src))


def test_init_without_gpu_fails_cleanly():
    import torch
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    with pytest.raises(le.LeError):
        le.Engine()


def test_gemm_workspace_size():
    L = qmm.lib()

    def gq(ty, m, k):  # fp16 activation fragments for m rounded up to 128, sum records, token scales
        mp = -(-m // 128) * 128
        srec = {12: 1024}.get(ty, 0)
        return mp * k * 2 + mp // 32 * (k // 256) * srec + mp * 4

    def gm(m, k):  # Q4_K split-activation GEMM: two fp16 planes + a 32-byte record per super-block
        return m * k * 4 + m * (k // 256) * 32

    assert L.le_gemm_workspace_size(12, 512, 4096) == max(gq(12, 512, 4096), gm(512, 4096))
    assert L.le_gemm_workspace_size(12, 1, 256) == max(gq(12, 1, 256), gm(1, 256))
    for ty in (8, 14, 16, 18):
        assert L.le_gemm_workspace_size(ty, 64, 4096) == gq(ty, 64, 4096)
    assert L.le_gemm_workspace_size(14, 64, 4096) == 128 * 4096 * 2 + 128 * 4
    assert L.le_gemm_workspace_size(12, 0, 4096) == 0
    assert L.le_gemm_workspace_size(12, 16, 100) == 0
    assert L.le_gemm_workspace_size(99, 16, 256) == 0
    # with room for up to 8 K slices' partial results (256-byte aligned) where a shape may split
    L.le_gemm_workspace_size_rows.restype = ctypes.c_size_t
    base = L.le_gemm_workspace_size(12, 64, 4096)
    assert L.le_gemm_workspace_size_rows(12, 64, 14336, 4096) == (base + 255) // 256 * 256 + 8 * 64 * 14336 * 4
    assert L.le_gemm_workspace_size_rows(14, 512, 200000, 4096) == L.le_gemm_workspace_size(14, 512, 4096)
    assert L.le_gemm_workspace_size_rows(12, 0, 4096, 4096) == 0


def test_moe_check_rejects_null_context():
    """le_moe_check validates its arguments on the host before touching the device."""
    L = qmm.lib()
    assert L.le_moe_check(None, None, None) == -1
    assert L.le_status_str(-8) == b"a bounded device-side wait gave up"
