"""Pins of the CPU oracle (oracle/le_oracle.c) against facts that do not come from the oracle itself.

The reference ships no golden vectors for this path (its only known-answer tests need an external
ik_llama build, src/quant_ik.rs:324-348, src/gpu.rs:692-737), and cannot be compiled here (Rust), so
each oracle function is pinned by mathematics and independent restatements:
  f16_to_f32      numpy's IEEE half conversion over all 65536 codes
  dequant         closed forms on hand-packed blocks (the packing below is written from the GGUF
                  block layouts, not from the oracle), scale/min recovery, sign patterns
  grids / ksign   value-set invariants, distinctness, even parity
  round trip      product quantizer -> oracle dequant error bounds (a transposed index or a wrong
                  nibble order gives ~140% error instead of a few %)
  matvec/matmat   bit-identity with numpy's strictly sequential float32 accumulate, float64 bound
  routing / MoE   numpy stable argsort, composition of matvecs
"""
import numpy as np
import pytest

import lastengine_amd as le
import oracle
from tests.util import weights, acts

F16_ONE = 0x3C00


def f16(x):
    return int(np.array(x, dtype=np.float16).view(np.uint16))


def test_f16_all_codes():
    codes = np.arange(65536, dtype=np.uint32)
    want = codes.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(c) for c in codes], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_ksign_even_parity():
    for i in range(128):
        s = oracle.ksign(i)
        assert s & 0x7F == i
        assert bin(s).count("1") % 2 == 0


def _grids():
    from oracle import HERE
    import os, re
    txt = open(os.path.join(HERE, "le_oracle_tables.h")).read()
    blocks = re.findall(r"\{([0-9,]+)\}", txt)
    g2 = np.array([[int(v) for v in b.split(",")] for b in blocks[:256]], dtype=np.int32)
    g3 = np.array([[int(v) for v in b.split(",")] for b in blocks[256:512]], dtype=np.int32)
    return g2, g3


def _grid_s():
    from oracle import HERE
    import os, re
    txt = open(os.path.join(HERE, "le_oracle_tables.h")).read()
    blocks = re.findall(r"\{([0-9,]+)\}", txt)
    return np.array([[int(v) for v in b.split(",")] for b in blocks[512:]], dtype=np.int32)


def test_iq2s_grid_invariants():
    """IQ2_S grid (src/quant_iq2_grids.rs:260-1284): 1024 distinct points with magnitudes in
    {8, 25, 43}, an even number of odd multiples of 8 per point, listed in strictly increasing order
    of the base-3 number whose digit j is the magnitude index of byte j (so a byte transposition or
    a dropped/duplicated row fails)."""
    gs = _grid_s()
    assert gs.shape == (1024, 8)
    assert set(np.unique(gs)) == {8, 25, 43}
    m = {8: 0, 25: 1, 43: 2}
    keys = [sum(m[int(v)] * 3 ** j for j, v in enumerate(r)) for r in gs]
    assert all(a < b for a, b in zip(keys, keys[1:]))
    assert set(((gs // 8) % 2).sum(1) % 2) == {0}


def test_grid_invariants():
    g2, g3 = _grids()
    assert g2.shape == (256, 8) and g3.shape == (256, 4)
    assert set(np.unique(g2)) == {8, 25, 43}
    assert set(np.unique(g3)) <= {4, 12, 20, 28, 36, 44, 52, 62}
    assert len({tuple(r) for r in g2}) == 256 and len({tuple(r) for r in g3}) == 256
    assert tuple(g2[0]) == (8,) * 8 and tuple(g3[0]) == (4,) * 4


def test_product_tables_match_oracle_tables():
    """The kernels' packed grid words carry the same magnitudes as the oracle's byte tables."""
    import os, re
    g2, g3 = _grids()
    txt = open(os.path.join(os.path.dirname(oracle.HERE), "lastengine_amd", "csrc", "le_iq_tables.h")).read()
    w2 = [int(v, 16) for v in re.findall(r"0x([0-9a-f]{8})u", txt.split("LE_IQ3XXS_GRID_WORDS")[0])]
    w3 = [int(v, 16) for v in re.findall(r"0x([0-9a-f]{8})u",
                                         txt.split("LE_IQ3XXS_GRID_WORDS")[1].split("LE_IQ2S_GRID_WORDS")[0])]
    ws = [int(v, 16) for v in re.findall(r"0x([0-9a-f]{8})u", txt.split("LE_IQ2S_GRID_WORDS")[1])]
    b2 = np.array(w2, dtype=np.uint32).view(np.uint8).reshape(256, 8)
    b3 = np.array(w3, dtype=np.uint32).view(np.uint8).reshape(256, 4)
    bs = np.array(ws, dtype=np.uint32).view(np.uint8).reshape(1024, 8)
    assert np.array_equal(b2, g2) and np.array_equal(b3, g3) and np.array_equal(bs, _grid_s())


# ---------------------------------------------------------------- closed forms

def test_q8_0_closed_form():
    rng = np.random.default_rng(1)
    blk = np.zeros((4, 34), dtype=np.uint8)
    d = [0.5, -0.0123, 3.0, 1e-6]
    q = rng.integers(-128, 128, size=(4, 32)).astype(np.int8)
    for i in range(4):
        blk[i, 0:2] = np.array([f16(d[i])], dtype=np.uint16).view(np.uint8)
        blk[i, 2:] = q[i].view(np.uint8)
    got = oracle.dequant_rows(8, blk.reshape(-1), 1, 128).reshape(4, 32)
    dd = np.array(d, dtype=np.float16).astype(np.float32)[:, None]
    assert np.array_equal(got, dd * q.astype(np.float32))


def _pack_k4(sc, m):
    """6-bit scales/mins into 12 bytes, written from the Q4_K/Q5_K layout description: the first
    four pairs live in the low 6 bits of bytes 0-3 (scales) and 4-7 (mins); pairs 4-7 keep their
    low nibbles in bytes 8-11 (scale low, min high) and their top two bits in bits 6-7 of bytes
    0-3 (scales) and 4-7 (mins)."""
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


def _q4k_block(d, dmin, sc, m, q):
    """q: 256 codes in value order. Value 64g+l is the low nibble of byte 32g+l, value 64g+32+l
    its high nibble."""
    b = np.zeros(144, dtype=np.uint8)
    b[0:2] = np.array([f16(d)], dtype=np.uint16).view(np.uint8)
    b[2:4] = np.array([f16(dmin)], dtype=np.uint16).view(np.uint8)
    b[4:16] = _pack_k4(sc, m)
    for g in range(4):
        for l in range(32):
            b[16 + 32 * g + l] = q[64 * g + l] | (q[64 * g + 32 + l] << 4)
    return b


def test_q4_k_closed_form_unit_scales():
    rng = np.random.default_rng(2)
    q = rng.integers(0, 16, size=256)
    blk = _q4k_block(0.75, 0.5, [1] * 8, [0] * 8, q)
    got = oracle.dequant_rows(12, blk, 1, 256)[0]
    assert np.array_equal(got, np.float32(0.75) * q.astype(np.float32))


def test_q4_k_scale_min_recovery():
    """Distinct 6-bit scales/mins for all eight sub-blocks (including the split high bits) are
    recovered from q=0 and q=15 rows."""
    sc = [63, 1, 37, 20, 45, 62, 17, 33]
    m = [5, 63, 0, 48, 31, 2, 59, 16]
    d, dmin = 0.25, 0.125
    lo = oracle.dequant_rows(12, _q4k_block(d, dmin, sc, m, [0] * 256), 1, 256)[0]
    hi = oracle.dequant_rows(12, _q4k_block(d, dmin, sc, m, [15] * 256), 1, 256)[0]
    for j in range(8):
        seg = slice(32 * j, 32 * j + 32)
        assert np.all(lo[seg] == -dmin * m[j])
        assert np.all(hi[seg] == d * sc[j] * 15 - dmin * m[j])


def _q6k_block(d, sc, q):
    """q: 256 codes (0..63) in value order. Value 128n + 32qd + l keeps its low 4 bits in ql and
    its top 2 bits in qh[32n+l] at bit 2qd. ql byte 64n+l holds quadrants 0 (low nibble) and 2
    (high nibble); ql byte 64n+32+l holds quadrants 1 and 3. Scale k (int8) covers values
    16k..16k+15; d f16 at byte 208."""
    b = np.zeros(210, dtype=np.uint8)
    for p in range(256):
        n, r = divmod(p, 128)
        qd, l = divmod(r, 32)
        idx = 64 * n + l + (32 if qd in (1, 3) else 0)
        b[idx] |= (q[p] & 15) << (4 if qd >= 2 else 0)
        b[128 + 32 * n + l] |= ((q[p] >> 4) & 3) << (2 * qd)
    b[192:208] = np.array(sc, dtype=np.int8).view(np.uint8)
    b[208:210] = np.array([f16(d)], dtype=np.uint16).view(np.uint8)
    return b


def test_q6_k_closed_form():
    rng = np.random.default_rng(3)
    q = rng.integers(0, 64, size=256)
    got = oracle.dequant_rows(14, _q6k_block(0.5, [1] * 16, q), 1, 256)[0]
    assert np.array_equal(got, np.float32(0.5) * (q - 32).astype(np.float32))
    sc = list(rng.integers(-128, 128, size=16))
    got = oracle.dequant_rows(14, _q6k_block(0.25, sc, [33] * 256), 1, 256)[0]
    assert np.array_equal(got, np.repeat(np.float32(0.25) * np.array(sc, dtype=np.float32), 16))


def test_iq2_xxs_grid0_and_signs():
    g2, _ = _grids()
    d = 0.5
    blk = np.zeros(66, dtype=np.uint8)
    blk[0:2] = np.array([f16(d)], dtype=np.uint16).view(np.uint8)
    sign_idx = [0, 1, 0x55, 127]
    grid_idx = [0, 7, 200, 255]
    for ib in range(8):
        s = ib * 2 % 16
        aux = s << 28
        for l in range(4):
            aux |= sign_idx[l] << (7 * l)
        blk[2 + 8 * ib: 6 + 8 * ib] = grid_idx
        blk[6 + 8 * ib: 10 + 8 * ib] = np.array([aux], dtype=np.uint32).view(np.uint8)
    got = oracle.dequant_rows(16, blk, 1, 256)[0]
    for ib in range(8):
        s = ib * 2 % 16
        db = np.float32(d) * np.float32(0.5 + s) * np.float32(0.25)
        for l in range(4):
            full = sign_idx[l] | ((bin(sign_idx[l]).count("1") & 1) << 7)
            sg = np.array([-1.0 if (full >> j) & 1 else 1.0 for j in range(8)], dtype=np.float32)
            want = db * g2[grid_idx[l]].astype(np.float32) * sg
            assert np.array_equal(got[32 * ib + 8 * l: 32 * ib + 8 * l + 8], want)


def test_iq3_xxs_grid_and_signs():
    _, g3 = _grids()
    d = 0.125
    blk = np.zeros(98, dtype=np.uint8)
    blk[0:2] = np.array([f16(d)], dtype=np.uint16).view(np.uint8)
    rng = np.random.default_rng(4)
    qs = rng.integers(0, 256, size=64)
    blk[2:66] = qs
    auxs = []
    for ib in range(8):
        aux = int(rng.integers(0, 1 << 28)) | ((15 - ib) << 28)
        auxs.append(aux)
        blk[66 + 4 * ib: 70 + 4 * ib] = np.array([aux], dtype=np.uint32).view(np.uint8)
    got = oracle.dequant_rows(18, blk, 1, 256)[0]
    for ib in range(8):
        db = np.float32(d) * np.float32(0.5 + (auxs[ib] >> 28)) * np.float32(0.5)
        for l in range(4):
            si = (auxs[ib] >> (7 * l)) & 127
            full = si | ((bin(si).count("1") & 1) << 7)
            mags = np.concatenate([g3[qs[8 * ib + 2 * l]], g3[qs[8 * ib + 2 * l + 1]]]).astype(np.float32)
            sg = np.array([-1.0 if (full >> j) & 1 else 1.0 for j in range(8)], dtype=np.float32)
            assert np.array_equal(got[32 * ib + 8 * l: 32 * ib + 8 * l + 8], db * mags * sg)


# ---------------------------------------------------------------- round trips

ROUNDTRIP_BOUND = {"Q8_0": 0.01, "Q4_K": 0.12, "Q6_K": 0.03, "IQ2_XXS": 0.5, "IQ3_XXS": 0.3}


@pytest.mark.parametrize("name", list(le.TYPES))
def test_quantize_dequant_roundtrip(name):
    ty = le.TYPES[name]
    q, src = weights(ty, 16, 2048, seed=11)
    got = oracle.dequant_rows(ty, q, 16, 2048)
    rel = np.sqrt(((got - src) ** 2).mean() / (src ** 2).mean())
    assert rel < ROUNDTRIP_BOUND[name], rel
    # correlation per row: a permuted layout would decorrelate
    for r in range(16):
        assert np.corrcoef(got[r], src[r])[0, 1] > 0.85


# ---------------------------------------------------------------- matvec / matmat / routing

@pytest.mark.parametrize("name", list(le.TYPES))
def test_matvec_sequential_sum(name):
    ty = le.TYPES[name]
    rows, cols = 24, 1024
    q, _ = weights(ty, rows, cols, seed=21)
    x = acts(cols, 22)
    y = oracle.matvec(ty, q, rows, cols, x)
    w = oracle.dequant_rows(ty, q, rows, cols)
    seq = np.add.accumulate(w * x[None, :], axis=1, dtype=np.float32)[:, -1]
    assert np.array_equal(y.view(np.uint32), seq.view(np.uint32))
    exact = (w.astype(np.float64) * x.astype(np.float64)).sum(axis=1)
    bound = cols * 2.0 ** -24 * (np.abs(w.astype(np.float64) * x)).sum(axis=1)
    assert np.all(np.abs(y - exact) <= bound)


def test_matmat_equals_matvec_columns():
    ty = le.Q4_K
    rows, cols = 40, 512
    q, _ = weights(ty, rows, cols, seed=31)
    xs = np.stack([acts(cols, 40 + t) for t in range(5)])
    Y = oracle.matmat(ty, q, rows, cols, xs, nthreads=3)
    for t in range(5):
        assert np.array_equal(Y[t], oracle.matvec(ty, q, rows, cols, xs[t], nthreads=1))


def test_route_matches_stable_argsort():
    for seed in range(20):
        lg = acts(128, 100 + seed)
        if seed == 0:
            lg[5] = lg[77] = lg.max() + 1.0  # a tie at the top: lower index first
        idx, w = oracle.route(lg, 8)
        z = lg.astype(np.float64) - lg.max()
        pr = np.exp(z) / np.exp(z).sum()
        order = np.argsort(-pr, kind="stable")[:8]
        assert list(idx) == list(order)
        np.testing.assert_allclose(w, pr[order] / pr[order].sum(), rtol=1e-5)
        if seed == 0:
            assert list(idx[:2]) == [5, 77]


def test_moe_composition():
    """Routed MoE = sum_s w_s * down_e(silu(gate_e h) * up_e h) with the oracle's own matvec."""
    n_exp, k, hidden, ff = 16, 4, 256, 256
    g, _ = weights(le.Q4_K, n_exp * ff, hidden, 51)
    u, _ = weights(le.Q4_K, n_exp * ff, hidden, 52)
    d, _ = weights(le.Q6_K, n_exp * hidden, ff, 53)
    h = np.stack([acts(hidden, 54), acts(hidden, 55)])
    lg = np.stack([acts(n_exp, 56), acts(n_exp, 57)])
    out, idx, w = oracle.moe(12, 12, 14, g, u, d, n_exp, k, hidden, ff, h, lg)
    rbg, rbd = le.row_bytes(12, hidden), le.row_bytes(14, ff)
    for t in range(2):
        i2, w2 = oracle.route(lg[t], k)
        assert list(i2) == list(idx[t])
        acc = np.zeros(hidden, dtype=np.float64)
        for s in range(k):
            e = idx[t, s]
            gg = oracle.matvec(12, g.reshape(-1)[e * ff * rbg:(e + 1) * ff * rbg], ff, hidden, h[t])
            uu = oracle.matvec(12, u.reshape(-1)[e * ff * rbg:(e + 1) * ff * rbg], ff, hidden, h[t])
            a = (gg / (1 + np.exp(-gg.astype(np.float64)))).astype(np.float32) * uu
            r = oracle.matvec(14, d.reshape(-1)[e * hidden * rbd:(e + 1) * hidden * rbd], hidden, ff, a)
            acc += w[t, s] * r.astype(np.float64)
        np.testing.assert_allclose(out[t], acc, rtol=1e-4, atol=1e-6)
