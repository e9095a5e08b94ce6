"""Pins of the oracle's wider formats (Q4_0, Q3_K, Q5_K, IQ2_S) and its int8 activation mode.

Each dequant is checked on blocks packed here from the GGUF block layout (the inverse direction of
the oracle's decoder, so a swapped nibble, a wrong bit of the high plane or a transposed scale index
fails), with power-of-two scales so the expected values are exact in float32.
quant_x is pinned by its defining properties (|x - d*q| <= d/2, max |q| = 127 at the block maximum,
xs = sum q), and matvec_q8 by a float64 dot of the oracle's own dequantized weights with the
dequantized activations d*q (a route that shares no code with udot's integer factorisation).
"""
import numpy as np
import pytest

import oracle

Q4_0, Q8_0, Q3_K, Q4_K, Q5_K, Q6_K, IQ2_XXS, IQ3_XXS, IQ2_S = 2, 8, 11, 12, 13, 14, 16, 18, 22
BLOCK = {Q4_0: (32, 18, [0]), Q8_0: (32, 34, [0]), Q3_K: (256, 110, [108]), Q4_K: (256, 144, [0, 2]),
         Q5_K: (256, 176, [0, 2]), Q6_K: (256, 210, [208]), IQ2_XXS: (256, 66, [0]), IQ3_XXS: (256, 98, [0]),
         IQ2_S: (256, 82, [0])}


def f16b(x):
    return np.array([x], dtype=np.float16).view(np.uint8)


def test_row_bytes_new_types():
    for ty, (v, b, _) in BLOCK.items():
        assert oracle.row_bytes(ty, 4096) == 4096 // v * b


def test_q4_0_closed_form():
    rng = np.random.default_rng(1)
    q = rng.integers(0, 16, size=(3, 32))
    d = [0.5, -0.25, 2.0]
    blk = np.zeros((3, 18), dtype=np.uint8)
    for i in range(3):
        blk[i, 0:2] = f16b(d[i])
        blk[i, 2:] = q[i, :16] | (q[i, 16:] << 4)   # value j: low nibble of byte j, j+16: high
    got = oracle.dequant_rows(Q4_0, blk.reshape(-1), 1, 96).reshape(3, 32)
    assert np.array_equal(got, np.array(d, dtype=np.float32)[:, None] * (q - 8).astype(np.float32))


def _pack_k4(sc, m):
    s = [0] * 12
    for j in range(8):
        if j < 4:
            s[j] |= sc[j] & 63
            s[j + 4] |= m[j] & 63
        else:
            s[j + 4] = (sc[j] & 15) | ((m[j] & 15) << 4)
            s[j - 4] |= (sc[j] >> 4) << 6
            s[j] |= (m[j] >> 4) << 6
    return s


def test_q5_k_closed_form():
    """Value 64g+l: low nibble of qs[32g+l] plus bit 2g of qh[l] as 16; value 64g+32+l: high
    nibble of the same byte plus bit 2g+1 (GGUF Q5_K: d, dmin, 12 scale bytes, qh[32], qs[128])."""
    rng = np.random.default_rng(2)
    q = rng.integers(0, 32, size=256)
    sc = [63, 1, 37, 20, 45, 62, 17, 33]
    m = [5, 63, 0, 48, 31, 2, 59, 16]
    d, dmin = 0.25, 0.125
    b = np.zeros(176, dtype=np.uint8)
    b[0:2], b[2:4], b[4:16] = f16b(d), f16b(dmin), _pack_k4(sc, m)
    for g in range(4):
        for l in range(32):
            lo, hi = q[64 * g + l], q[64 * g + 32 + l]
            b[48 + 32 * g + l] = (lo & 15) | ((hi & 15) << 4)
            b[16 + l] |= ((lo >> 4) << (2 * g)) | ((hi >> 4) << (2 * g + 1))
    got = oracle.dequant_rows(Q5_K, b, 1, 256)[0]
    want = np.array([d * sc[e // 32] * q[e] - dmin * m[e // 32] for e in range(256)], dtype=np.float32)
    assert np.array_equal(got, want)


def test_q3_k_closed_form():
    """GGUF Q3_K: hmask[32], qs[64], 12 scale bytes, d. Value e = 128c + 32s + l takes 2 bits at
    2s of qs[32c+l] and bit e//32 of hmask[l] (clear = subtract 4); 16 signed 6-bit scales (stored
    +32): low nibbles of scale bytes 0-7 for 0-7 and their high nibbles for 8-15, top two bits of
    scale i at bits 2(i//4) of byte 8 + i%4."""
    rng = np.random.default_rng(3)
    q = rng.integers(-4, 4, size=256)
    scales = rng.integers(-32, 32, size=16)
    d = 0.5
    b = np.zeros(110, dtype=np.uint8)
    for e in range(256):
        c, s, l = e // 128, (e % 128) // 32, e % 32
        v = q[e] + 4 if q[e] < 0 else q[e]
        hb = 0 if q[e] < 0 else 1
        b[32 + 32 * c + l] |= (v & 3) << (2 * s)
        b[l] |= hb << (e // 32)
    for i in range(16):
        u = int(scales[i]) + 32
        if i < 8:
            b[96 + i] |= u & 15
        else:
            b[96 + i - 8] |= (u & 15) << 4
        b[96 + 8 + i % 4] |= (u >> 4) << (2 * (i // 4))
    b[108:110] = f16b(d)
    got = oracle.dequant_rows(Q3_K, b, 1, 256)[0]
    want = np.array([d * scales[e // 16] * q[e] for e in range(256)], dtype=np.float32)
    assert np.array_equal(got, want)


def _grid_s():
    import os, re
    txt = open(os.path.join(oracle.HERE, "le_oracle_tables.h")).read()
    blocks = re.findall(r"\{([0-9,]+)\}", txt)
    return np.array([[int(v) for v in b.split(",")] for b in blocks[512:]], dtype=np.int32)


def test_iq2_s_grid_and_signs():
    """GGUF IQ2_S: d, qs[32] (low 8 index bits), signs[32] (one explicit sign byte per 8 values),
    qh[8] (two high index bits per group of 8 at bits 2l), scales[8] (low nibble: groups 0-1,
    high: 2-3); value scale d * (0.5 + s) / 4."""
    gs = _grid_s()
    rng = np.random.default_rng(5)
    d = 0.125
    gi = rng.integers(0, 1024, size=32)
    gi[0], gi[1] = 0, 1023
    sg = rng.integers(0, 256, size=32)
    sc = rng.integers(0, 256, size=8)
    b = np.zeros(82, dtype=np.uint8)
    b[0:2] = f16b(d)
    for k in range(32):
        ib, l = divmod(k, 4)
        b[2 + k] = gi[k] & 255
        b[34 + k] = sg[k]
        b[66 + ib] |= (gi[k] >> 8) << (2 * l)
    b[74:82] = sc
    got = oracle.dequant_rows(IQ2_S, b, 1, 256)[0]
    for k in range(32):
        ib, l = divmod(k, 4)
        s = (sc[ib] & 15) if l < 2 else (sc[ib] >> 4)
        db = np.float32(d) * np.float32(0.5 + s) * np.float32(0.25)
        sign = np.array([-1.0 if (sg[k] >> j) & 1 else 1.0 for j in range(8)], dtype=np.float32)
        assert np.array_equal(got[8 * k: 8 * k + 8], db * gs[gi[k]].astype(np.float32) * sign), k


def test_quant_x_properties():
    rng = np.random.default_rng(7)
    x = rng.normal(size=32 * 64).astype(np.float32)
    x[32:64] = 0.0                                 # an all-zero block: d = 0, q = 0
    x[64:96] *= 1e-30                              # tiny values
    x[96:128] *= 1e4
    xq, xd, xs = oracle.quant_x(x)
    xb = x.reshape(-1, 32)
    qb = xq.reshape(-1, 32).astype(np.int64)
    amax = np.abs(xb).max(axis=1)
    np.testing.assert_array_equal(xd, (amax / np.float32(127)).astype(np.float32))
    assert np.all(np.abs(qb) <= 127)
    np.testing.assert_array_equal(xs, qb.sum(axis=1))
    err = np.abs(xb.astype(np.float64) - xd[:, None].astype(np.float64) * qb)
    assert np.all(err <= 0.5 * xd[:, None] * (1 + 1e-6) + 1e-45)
    live = amax > 0
    top = np.abs(xb).argmax(axis=1)
    assert np.all(np.abs(qb[np.arange(len(qb)), top])[live] == 127)
    assert np.all(qb[1] == 0) and xd[1] == 0


def _random_blocks(ty, rows, cols, seed):
    v, bb, offs = BLOCK[ty]
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 256, size=(rows, cols // v, bb), dtype=np.uint8)
    for o in offs:
        q[:, :, o:o + 2] = rng.uniform(-0.01, 0.01, size=(rows, cols // v)).astype(np.float16).view(
            np.uint8).reshape(rows, cols // v, 2)
    return q.reshape(rows, -1)


@pytest.mark.parametrize("ty", sorted(BLOCK))
@pytest.mark.parametrize("cols", [768, 4096])
def test_matvec_q8_vs_float64(ty, cols):
    rows = 12
    w = _random_blocks(ty, rows, cols, seed=ty * 100 + cols)
    x = np.random.default_rng(cols + ty).normal(size=cols).astype(np.float32)
    xq, xd, xs = oracle.quant_x(x)
    y = oracle.matvec_q8(ty, w, rows, cols, xq, xd, xs)
    wd = oracle.dequant_rows(ty, w, rows, cols).astype(np.float64)
    xa = np.repeat(xd.astype(np.float64), 32) * xq.astype(np.float64)
    exact = wd @ xa
    mag = np.abs(wd) @ np.abs(xa)
    assert np.all(np.abs(y - exact) <= 64 * 2.0 ** -24 * mag + 1e-30), np.max(np.abs(y - exact) / mag)
    # and the int8 mode tracks the fp32 oracle within the activation quantization error
    yf = oracle.matvec(ty, w, rows, cols, x)
    assert np.all(np.abs(y - yf) <= 0.02 * (np.abs(wd) @ np.abs(x.astype(np.float64))) + 1e-30)


def test_rms_pins():
    """or_rms against numpy: the strictly sequential float32 sum of squares (bit-identical), and
    the float64 RMSNorm within a few ulp; constant input has the closed form w * c / sqrt(c^2 + eps)."""
    rng = np.random.default_rng(11)
    x = rng.normal(size=4096).astype(np.float32)
    w = rng.normal(size=4096).astype(np.float32)
    o = oracle.rms(x, w, 1e-6)
    ss = np.add.accumulate(x * x, dtype=np.float32)[-1] / np.float32(4096)
    r = np.float32(1.0) / np.sqrt(ss + np.float32(1e-6))
    assert np.array_equal(o, (x * r) * w)
    ref = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean() + 1e-6) * w
    assert np.allclose(o, ref, rtol=1e-5, atol=1e-6)
    c = np.full(64, 3.0, dtype=np.float32)
    np.testing.assert_allclose(oracle.rms(c, np.ones(64, np.float32), 0.0), np.ones(64), rtol=1e-6)


def test_swiglu_pins():
    """or_swiglu against a float64 silu(g) * u within float32 rounding, and its closed forms
    (silu(0) = 0, silu(g) -> g for large g, -> 0 for very negative g)."""
    rng = np.random.default_rng(12)
    g = (rng.normal(size=4096) * 4).astype(np.float32)
    u = rng.normal(size=4096).astype(np.float32)
    o = oracle.swiglu(g, u)
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.allclose(o, ref, rtol=2e-6, atol=1e-30)
    z = oracle.swiglu(np.array([0.0, 60.0, -60.0], np.float32), np.ones(3, np.float32))
    assert z[0] == 0.0 and z[1] == np.float32(60.0) and abs(z[2]) < 1e-20
