"""GGUF reader (include/le_gguf.h) on files written by tests/gguf_writer.py: header, every kv value
type with the reference's as_u64 / as_f32 / as_str meanings (src/gguf.rs:14-24), tensor infos,
data start alignment, expert slabs of 3D tensors (src/cpu_ref.rs:70-85), raw reads, and the
reference's rejections (bad magic, version, counts, dims, truncation; src/gguf.rs:97-117)."""
import struct

import numpy as np
import pytest

import lastengine_amd as le
from lastengine_amd.gguf import Gguf
from tests import gguf_writer as W


def _kv():
    return [("general.architecture", W.STR, "qwen3moe"),
            ("general.alignment", W.U32, 64),
            ("qwen3moe.block_count", W.U32, 48),
            ("qwen3moe.expert_count", W.U64, 128),
            ("qwen3moe.expert_used_count", W.I32, 8),
            ("neg", W.I16, -5),
            ("small", W.U8, 7), ("tiny", W.I8, 3), ("mid", W.U16, 512),
            ("flag", W.BOOL, 1),
            ("eps", W.F32, 1e-6), ("base", W.F64, 1000000.0),
            ("big", W.I64, 1 << 40),
            ("tokens", W.ARR, (W.STR, ["<s>", "</s>", "hello"])),
            ("nested", W.ARR, (W.ARR, [(W.U32, [1, 2]), (W.U32, [3])])),
            ("scores", W.ARR, (W.F32, [0.5, -1.0]))]


def _tensors():
    rng = np.random.default_rng(0)
    ty_g, ty_d = le.Q4_K, le.Q6_K
    g = rng.integers(0, 256, size=4 * 16 * le.row_bytes(ty_g, 512), dtype=np.uint8)    # 4 experts x 16 rows x 512
    d = rng.integers(0, 256, size=4 * 512 * le.row_bytes(ty_d, 256), dtype=np.uint8)   # 4 experts x 512 rows x 256
    q8 = rng.integers(0, 256, size=3 * le.row_bytes(le.Q8_0, 64), dtype=np.uint8)
    f32 = np.arange(10, dtype=np.float32).view(np.uint8)
    return [("blk.0.ffn_gate_exps.weight", [512, 16, 4], ty_g, g),
            ("blk.0.ffn_down_exps.weight", [256, 512, 4], ty_d, d),
            ("output.weight", [64, 3], le.Q8_0, q8),
            ("norm.weight", [10], 0, f32)]


@pytest.fixture(scope="module")
def gfile(tmp_path_factory):
    p = tmp_path_factory.mktemp("g") / "m.gguf"
    offs = W.write(str(p), _kv(), _tensors(), alignment=64)
    return str(p), offs


def test_header_and_kv(gfile):
    g = Gguf(gfile[0])
    assert g.version == 3 and g.kv_count == len(_kv()) and len(g.tensors) == 4
    assert g.arch() == "qwen3moe"
    assert g.as_u64("qwen3moe.block_count") == 48 and g.as_u64("qwen3moe.expert_count") == 128
    assert g.as_u64("qwen3moe.expert_used_count") == 8          # non-negative signed -> u64
    assert g.as_u64("neg") is None and g.as_i64("neg") == -5    # negative signed: no u64
    assert g.as_u64("small") == 7 and g.as_u64("tiny") == 3 and g.as_u64("mid") == 512
    assert g.as_u64("flag") == 1                                # bool -> u64
    assert g.as_u64("big") == 1 << 40
    assert g.as_f32("eps") == np.float32(1e-6) and g.as_f32("base") == 1e6
    assert g.as_f32("small") is None and g.as_str("eps") is None and g.as_u64("eps") is None
    assert g.array("tokens") == (W.STR, 3) and g.array("nested") == (W.ARR, 2) and g.array("scores") == (W.F32, 2)
    assert g.kv_type("missing") == -1 and g.kv_type("base") == W.F64


def test_tensor_infos_and_alignment(gfile):
    path, offs = gfile
    g = Gguf(path)
    assert g.data_start % 64 == 0
    for (name, dims, ty, raw), t, off in zip(_tensors(), g.tensors, offs):
        assert t.name == name and t.dims == dims and t.ggml_type == ty and t.offset == off
        if ty != 0:
            assert t.nbytes == len(raw)
        assert np.array_equal(g.read(t.offset, len(raw)), raw)
    assert g.find("nope") is None
    assert g.tensors[3].nbytes == 0  # f32 (type 0) is not a quantized type of this build


def test_expert_slabs(gfile):
    g = Gguf(gfile[0])
    raw = dict((n, r) for n, _, _, r in _tensors())
    for name in ("blk.0.ffn_gate_exps.weight", "blk.0.ffn_down_exps.weight"):
        t = g.find(name)
        slab = len(raw[name]) // 4
        for e in range(4):
            off, nb = g.expert_slab(name, e)
            assert nb == slab and off == t.offset + e * slab
            assert np.array_equal(g.read(off, nb), raw[name][e * slab:(e + 1) * slab])
        with pytest.raises(le.LeError):
            g.expert_slab(name, 4)
    off, nb = g.expert_slab("output.weight", 0)   # 2D tensor: expert 0 is the whole tensor
    assert nb == le.row_bytes(le.Q8_0, 64) * 3
    with pytest.raises(le.LeError):
        g.read(g.tensors[-1].offset, 1 << 30)     # past the end of the file


def _bad(tmp_path, data):
    p = tmp_path / "bad.gguf"
    p.write_bytes(data)
    with pytest.raises(le.LeError) as e:
        Gguf(str(p))
    return str(e.value)


def test_rejections(tmp_path, gfile):
    good = open(gfile[0], "rb").read()
    assert "not a GGUF file" in _bad(tmp_path, b"GGUX" + good[4:])
    assert "unsupported GGUF version" in _bad(tmp_path, good[:4] + struct.pack("<I", 1) + good[8:])
    assert "implausible counts" in _bad(tmp_path, good[:8] + struct.pack("<Q", (1 << 24) + 1) + good[16:])
    assert "truncated" in _bad(tmp_path, good[:200])
    p = tmp_path / "dims.gguf"
    W.write(str(p), [], [("t", [1] * 9, le.Q8_0, np.zeros(34, np.uint8))])
    with pytest.raises(le.LeError) as e:
        Gguf(str(p))
    assert "too many dims" in str(e.value)
    p2 = tmp_path / "ty.gguf"
    blob = bytearray(b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + W._str("k") + struct.pack("<I", 13) + b"\0" * 8)
    p2.write_bytes(bytes(blob))
    with pytest.raises(le.LeError) as e:
        Gguf(str(p2))
    assert "unknown value type" in str(e.value)


def test_v2_and_default_alignment(tmp_path):
    p = tmp_path / "v2.gguf"
    offs = W.write(str(p), [("a", W.STR, "x")], [("w", [64, 2], le.Q8_0, np.arange(136, dtype=np.uint8))],
                   alignment=32, version=2)
    g = Gguf(str(p))
    assert g.version == 2 and g.data_start % 32 == 0 and g.tensors[0].offset == offs[0]


def test_tensor_extent_checks(tmp_path):
    """A tensor whose dims product overflows 64 bits, or whose data would run past the end of the
    file, is reported as an error (LE_ERR_SHAPE) by le_gguf_tensor_info and le_gguf_expert_slab
    instead of a wrapped size or an out-of-file offset; the other tensors stay readable."""
    ok = np.arange(34 * 2, dtype=np.uint8)
    tensors = [("ok", [64], le.Q8_0, ok),
               ("wrap", [1 << 40, 1 << 40, 1 << 20], le.Q8_0, ok[:34]),   # 2^100 values: the product wraps
               ("past_end", [32, 1000, 4], le.Q8_0, ok[:34])]             # 136000 bytes claimed, 34 present
    p = tmp_path / "bad.gguf"
    W.write(str(p), [("general.architecture", W.STR, "llama")], tensors, alignment=32)
    g = Gguf(str(p))
    assert g.find("ok").fits and g.find("ok").nbytes == 68
    assert np.array_equal(g.tensor_bytes("ok"), ok)
    for name in ("wrap", "past_end"):
        t = g.find(name)
        assert not t.fits and t.nbytes == 0
        with pytest.raises(le.LeError) as e:
            g.tensor_bytes(name)
        assert e.value.code == -3
        with pytest.raises(le.LeError) as e:
            g.expert_slab(name, 0)
        assert e.value.code == -3
