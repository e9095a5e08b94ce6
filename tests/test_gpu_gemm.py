"""GPU parity of the matrix-core GEMM (le_gemm from the token count where it takes over) for every
type, against the oracle's cpu_ref::matmat restatement (src/cpu_ref.rs:266-276).

Bar (tests/util.py): max|got-want| / max|want| <= 1e-3 and |got-want| <= 1e-3 * sum|w*x| per
output. Weights enter the matrix cores as exact integer codes (Q4_K, Q5_K, Q3_K, IQ2_XXS, IQ3_XXS,
IQ2_S; Q6_K where the code has at most 11 significant bits) or rounded once to fp16 (Q6_K otherwise,
Q8_0, Q4_0), and activations as fp16 after a per-token power-of-two scale (relative error 2^-11).
The types without a quantizer here (Q4_0, Q3_K, Q5_K, IQ2_S) are tested on arbitrary block bytes
with bounded finite scales."""
import numpy as np
import pytest

import lastengine_amd as le
import oracle
from tests.util import weights, acts, check_close, random_blocks, wbytes

pytestmark = pytest.mark.gpu

NAMES = list(le.MV_TYPES)
# Full-size weights of the configs: Q4_K / IQ2_XXS gate-up, Q6_K / IQ3_XXS down, Q8_0 head; the other
# formats at the gate/up shape
FULL = {"Q4_K": (14336, 4096), "Q6_K": (4096, 14336), "Q8_0": (32000, 4096), "IQ2_XXS": (14336, 4096),
        "IQ3_XXS": (4096, 14336), "Q4_0": (14336, 4096), "Q3_K": (14336, 4096), "Q5_K": (14336, 4096),
        "IQ2_S": (14336, 4096)}


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def run_gemm(engine, ty, q, xs, rows, cols):
    import torch
    m = xs.shape[0]
    y = torch.full((m, rows), float("nan"), dtype=torch.float32, device="cuda")
    engine.gemm(ty, dev(q), dev(xs), m, y, rows, cols)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def absmag(ty, q, rows, cols, xs):
    w = oracle.dequant_rows(ty, q, rows, cols).astype(np.float32)
    return (np.abs(xs).astype(np.float32) @ np.abs(w).T).astype(np.float64)


@pytest.mark.parametrize("name", NAMES)
@pytest.mark.parametrize("m", [17, 64, 512])
def test_gemm_full_shapes(engine, name, m):
    ty = le.MV_TYPES[name]
    rows, cols = FULL[name]
    print("gemm full", name, rows, cols, m, flush=True)
    q = wbytes(ty, rows, cols, seed=40 + ty)
    xs = np.stack([acts(cols, 7000 + t) for t in range(m)])
    got = run_gemm(engine, ty, q, xs, rows, cols)
    want = oracle.matmat(ty, q, rows, cols, xs)
    check_close(got, want, absmag(ty, q, rows, cols, xs))


@pytest.mark.parametrize("name", NAMES)
@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5, 6, 7, 8, 9, 10])
@pytest.mark.parametrize("rows,cols,m,ks", [(300, 512, 17, 0), (513, 768, 65, 1), (96, 4096, 40, 4), (1000, 1024, 130, 2)])
def test_gemm_tiles_and_slices(fresh_engine, name, cfg, rows, cols, m, ks):
    """Every block shape (32/64/128 tokens x 128/256 rows, 4 or 8 waves) with ragged row and token tiles and
    explicit K slices (fp32 atomic adds into the cleared output)."""
    engine = fresh_engine
    engine.set_option("gq_cfg", cfg)
    engine.set_option("gq_ksplit", ks)
    engine.set_option("gq_min_m", 1)
    engine.set_option("gm_min_m", 1)
    engine.set_option("gm_mh", 0)
    ty = le.MV_TYPES[name]
    if (cols // 256) % max(ks, 1):
        pytest.skip("K slices must divide the super-blocks")
    print("gemm tiles", name, cfg, rows, cols, m, ks, flush=True)
    q = wbytes(ty, rows, cols, seed=rows + m + ty)
    xs = np.stack([acts(cols, 8000 + t) for t in range(m)])
    got = run_gemm(engine, ty, q, xs, rows, cols)
    want = oracle.matmat(ty, q, rows, cols, xs)
    check_close(got, want, absmag(ty, q, rows, cols, xs))


@pytest.mark.parametrize("cfg", [11, 12])
@pytest.mark.parametrize("rows,cols,m,ks", [(300, 512, 17, 0), (513, 768, 65, 1), (96, 4096, 40, 4), (1000, 1024, 130, 2), (700, 2048, 300, 0)])
def test_gemm_q4k_wave_grid_tiles(fresh_engine, cfg, rows, cols, m, ks):
    """The Q4_K tiles on 2 x 4 waves (cfg 11: 128 x 256, waves of 64 x 64; cfg 12: 128 x 128, waves
    of 64 x 32), with ragged tiles and K slices."""
    engine = fresh_engine
    engine.set_option("gq_cfg", cfg)
    engine.set_option("gq_ksplit", ks)
    engine.set_option("gm_min_m", 1)
    engine.set_option("gm_mh", 0)
    ty = le.Q4_K
    if (cols // 256) % max(ks, 1):
        pytest.skip("K slices must divide the super-blocks")
    print("gemm q4k wave grid", cfg, rows, cols, m, ks, flush=True)
    q = wbytes(ty, rows, cols, seed=rows + m + 5)
    xs = np.stack([acts(cols, 8100 + t) for t in range(m)])
    got = run_gemm(engine, ty, q, xs, rows, cols)
    check_close(got, oracle.matmat(ty, q, rows, cols, xs), absmag(ty, q, rows, cols, xs))


@pytest.mark.parametrize("name", NAMES)
@pytest.mark.parametrize("m", [1, 8, 24, 96])
def test_gemm_random_blocks(engine, name, m):
    """Arbitrary block bytes with bounded finite scales: every 6-bit scale/min code, negative Q6_K
    sub-block scales, every IQ grid index and sign pattern, on the vector and matrix-core paths."""
    ty = le.MV_TYPES[name]
    rows, cols = 384, 2048
    print("gemm random blocks", name, m, flush=True)
    q = random_blocks(ty, rows, cols, seed=11 * ty + m)
    xs = np.stack([acts(cols, 9000 + t) for t in range(m)])
    got = run_gemm(engine, ty, q, xs, rows, cols)
    want = oracle.matmat(ty, q, rows, cols, xs)
    check_close(got, want, absmag(ty, q, rows, cols, xs))


@pytest.mark.parametrize("name", NAMES)
@pytest.mark.parametrize("m", [5, 12, 40])
def test_gemm_activation_magnitudes(engine, name, m):
    """Tokens of very different magnitude in one call (1e-6 .. 1e6, a zero token, one token with a
    single non-zero value): each token (3..16-token Q4_K kernel: each token's super-block) is
    scaled by its own power of two before fp16, so none overflows and none loses relative
    precision."""
    if m < 9 and name != "Q4_K":
        pytest.skip("below 9 tokens the other types run on the vector kernels (per-block int8 images, "
                    "no fp16 range); their offset form leaves 2^-15-level residues where sum|wx| is 0")
    ty = le.MV_TYPES[name]
    rows, cols = 256, 1024
    zt, st = (3, 7) if m > 7 else (1, m - 1)
    q = wbytes(ty, rows, cols, seed=5 + ty)
    xs = np.stack([acts(cols, 9500 + t) for t in range(m)])
    scales = np.float32(10.0) ** np.linspace(-6, 6, m).astype(np.float32)
    xs = (xs * scales[:, None]).astype(np.float32)
    xs[zt] = 0.0
    xs[st] = 0.0
    xs[st, 100] = 3.0e4
    print("gemm magnitudes", name, m, flush=True)
    got = run_gemm(engine, ty, q, xs, rows, cols)
    want = oracle.matmat(ty, q, rows, cols, xs)
    mag = absmag(ty, q, rows, cols, xs)
    assert np.all(got[zt] == 0.0)
    # per token: the bar relative to that token's own outputs
    for t in range(m):
        if t == zt:
            continue
        check_close(got[t:t + 1], want[t:t + 1], mag[t:t + 1])


@pytest.mark.parametrize("name", NAMES)
@pytest.mark.parametrize("rows,cols,m,ks", [(1000, 4096, 64, 4), (257, 2048, 20, 8), (130, 1024, 33, 2)])
def test_gemm_slice_sums(fresh_engine, name, rows, cols, m, ks):
    """K slices with the partial-result workspace (le_gemm_workspace_size_rows: summed in a second
    pass, slice order fixed) and with the minimal one (atomic adds into y): both meet the oracle
    bar, and the summed form gives the same bits on a second call."""
    import torch
    ty = le.MV_TYPES[name]
    fresh_engine.set_option("gq_ksplit", ks)
    if name == "Q4_K":
        fresh_engine.set_option("gm_min_m", 17)
        fresh_engine.set_option("gm_mh", 0)
    q = wbytes(ty, rows, cols, seed=ks + m)
    xs = acts(m * cols, seed=rows).reshape(m, cols)
    want = oracle.matmat(ty, q, rows, cols, xs)
    mag = absmag(ty, q, rows, cols, xs)
    dq, dx = dev(q), dev(xs)
    full = fresh_engine.gemm_workspace_size_rows(ty, m, rows, cols)
    small = fresh_engine.gemm_workspace_size(ty, m, cols)
    assert full >= small + ks * m * rows * 4
    outs = []
    for nbytes in (full, full, small):
        print("slice sums", name, rows, cols, m, ks, nbytes, flush=True)
        ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        y = torch.full((m, rows), float("nan"), dtype=torch.float32, device="cuda")
        fresh_engine.gemm(ty, dq, dx, m, y, rows, cols, ws=ws)
        torch.cuda.synchronize()
        outs.append(y.cpu().numpy())
        check_close(outs[-1], want, mag)
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


@pytest.mark.parametrize("name", ["Q8_0", "Q4_0"])
@pytest.mark.parametrize("m", [17, 130])
def test_gemm_per_block_scale_range(engine, name, m):
    """Q8_0 / Q4_0 carry a scale per 32 values inside their fp16 codes: blocks with |d| from 2^-20
    to 3e4 in one row (fp16 scales up to the top of its range, and codes that would leave it under
    a fixed multiplier) and a row of all-zero scales stay within the parity bar."""
    ty = le.MV_TYPES[name]
    rows, cols = 200, 2048
    q = random_blocks(ty, rows, cols, seed=300 + m)
    bb = 34 if ty == le.Q8_0 else 18
    blk = q.reshape(rows, -1, bb)
    rng = np.random.default_rng(m)
    mag = np.float32(2.0) ** rng.uniform(-20, np.log2(3.0e4), size=blk.shape[:2]).astype(np.float32)
    d = (mag * rng.choice([-1, 1], size=blk.shape[:2])).astype(np.float16)
    d[5] = 0
    blk[:, :, 0:2] = d.view(np.uint8).reshape(rows, -1, 2)
    xs = np.stack([acts(cols, 9100 + t) for t in range(m)])
    print("gemm scale range", name, m, flush=True)
    got = run_gemm(engine, ty, q, xs, rows, cols)
    want = oracle.matmat(ty, q, rows, cols, xs)
    assert np.all(got[:, 5] == 0.0)
    check_close(got, want, absmag(ty, q, rows, cols, xs))
