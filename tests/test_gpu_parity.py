"""GPU parity: the HIP path (through the C ABI) against the CPU oracle on identical seeded inputs.

Bars: dequantized weights bit-exact; matvec/GEMM outputs within max|d|/max|want| <= 1e-3 and
|d| <= 1e-3 * sum|w*x| per output (tests/util.py)."""
import numpy as np
import pytest

import lastengine_amd as le
import oracle
from tests.util import weights, acts, check_close

pytestmark = pytest.mark.gpu

NAMES = list(le.TYPES)


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def sync():
    import torch
    torch.cuda.synchronize()


def absmag(ty, q, rows, cols, xs):
    w = oracle.dequant_rows(ty, q, rows, cols).astype(np.float64)
    return np.abs(np.atleast_2d(xs).astype(np.float64)) @ np.abs(w).T


# ------------------------------------------------------------------ dequant

@pytest.mark.parametrize("name", NAMES)
@pytest.mark.parametrize("rows,cols", [(8, 1024), (37, 2048), (3, 4096)])
def test_dequant_bit_exact(engine, name, rows, cols):
    import torch
    ty = le.TYPES[name]
    q, _ = weights(ty, rows, cols, seed=rows * 1000 + cols)
    out = torch.empty(rows, cols, dtype=torch.float32, device="cuda")
    engine.dequant_rows(ty, dev(q), out, rows, cols)
    sync()
    want = oracle.dequant_rows(ty, q, rows, cols)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("name", NAMES)
def test_dequant_random_bytes_bit_exact(engine, name):
    """Arbitrary block bytes, including f16 scales that are subnormal, Inf or NaN. Every non-NaN
    value is bit-identical; NaN results must be NaN (arithmetic NaN payloads are not portable:
    x86 returns the negative default NaN where the GPU returns the positive canonical one)."""
    import torch
    ty = le.TYPES[name]
    rows, cols = 16, 1024
    rng = np.random.default_rng(ty)
    q = rng.integers(0, 256, size=(rows, le.row_bytes(ty, cols)), dtype=np.uint8)
    out = torch.empty(rows, cols, dtype=torch.float32, device="cuda")
    engine.dequant_rows(ty, dev(q), out, rows, cols)
    sync()
    want = oracle.dequant_rows(ty, q, rows, cols)
    got = out.cpu().numpy()
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


# ------------------------------------------------------------------ matvec

@pytest.mark.parametrize("name", NAMES)
@pytest.mark.parametrize("rows,cols", [(64, 256), (100, 1024), (333, 4096), (77, 768), (40, 14336), (1, 512)])
def test_matvec_parity(engine, name, rows, cols):
    import torch
    ty = le.TYPES[name]
    q, _ = weights(ty, rows, cols, seed=rows + cols + ty)
    x = acts(cols, seed=cols + 7)
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    engine.mv(ty, dev(q), dev(x), y, rows, cols)
    sync()
    want = oracle.matvec(ty, q, rows, cols, x)
    check_close(y.cpu().numpy(), want, absmag(ty, q, rows, cols, x)[0])


def test_matvec_slots_ptr_table(engine):
    """mv_ptrs semantics: slot s reads ptrs[s] and x + s*xstride, writes y[s*rows:]."""
    import torch
    ty, rows, cols, slots = le.Q4_K, 96, 2048, 3
    qs = [weights(ty, rows, cols, seed=500 + s)[0] for s in range(slots)]
    xs = np.stack([acts(cols, 600 + s) for s in range(slots)])
    bufs = [dev(q) for q in qs]
    ptrs = torch.tensor([b.data_ptr() for b in bufs], dtype=torch.int64, device="cuda")
    y = torch.empty(slots * rows, dtype=torch.float32, device="cuda")
    engine.mv_ptrs(ty, ptrs, dev(xs), y, rows, cols, cols, slots)
    sync()
    got = y.cpu().numpy().reshape(slots, rows)
    for s in range(slots):
        check_close(got[s], oracle.matvec(ty, qs[s], rows, cols, xs[s]), absmag(ty, qs[s], rows, cols, xs[s])[0])
    # shared activation (xstride = 0) over a contiguous slab (no pointer table)
    slab = np.concatenate(qs, axis=0)
    y2 = torch.empty(slots * rows, dtype=torch.float32, device="cuda")
    engine.mv_ptrs(ty, None, dev(xs[0]), y2, rows, cols, 0, slots, w=dev(slab))
    sync()
    got = y2.cpu().numpy().reshape(slots, rows)
    for s in range(slots):
        check_close(got[s], oracle.matvec(ty, qs[s], rows, cols, xs[0]), absmag(ty, qs[s], rows, cols, xs[0])[0])


# configs 1, 2 (including the concatenated gate+up matrix) and 5 at their full sizes
FULL = [("Q4_K", 4096, 4096), ("Q4_K", 14336, 4096), ("Q4_K", 28672, 4096), ("Q4_K", 1024, 4096), ("Q6_K", 4096, 14336),
        ("Q8_0", 32000, 4096), ("IQ2_XXS", 14336, 4096), ("IQ3_XXS", 4096, 14336)]


@pytest.mark.parametrize("name,rows,cols", FULL)
def test_matvec_config_sizes(engine, name, rows, cols):
    import torch
    ty = le.TYPES[name]
    q, _ = weights(ty, rows, cols, seed=rows * 7 + cols)
    x = acts(cols, seed=cols)
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    engine.mv(ty, dev(q), dev(x), y, rows, cols)
    sync()
    want = oracle.matvec(ty, q, rows, cols, x)
    check_close(y.cpu().numpy(), want, absmag(ty, q, rows, cols, x)[0])


@pytest.mark.parametrize("name,rows,cols", FULL)
def test_matvec_config_sizes_random_blocks(engine, name, rows, cols):
    """The config shapes on arbitrary block bytes with bounded finite scales (every scale/min code,
    negative Q6_K scales, every IQ grid index and sign pattern) through the staged kernels."""
    import torch
    from tests.util import random_blocks
    ty = le.TYPES[name]
    q = random_blocks(ty, rows, cols, seed=rows + cols + ty)
    x = acts(cols, seed=cols + 1)
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    engine.mv(ty, dev(q), dev(x), y, rows, cols)
    sync()
    want = oracle.matvec(ty, q, rows, cols, x)
    check_close(y.cpu().numpy(), want, absmag(ty, q, rows, cols, x)[0])


# ------------------------------------------------------------------ small-M GEMM

@pytest.mark.parametrize("name", NAMES)
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 13, 16])
def test_gemm_small_m(engine, name, m):
    import torch
    ty = le.TYPES[name]
    rows, cols = 200, 1024
    q, _ = weights(ty, rows, cols, seed=900 + ty)
    xs = np.stack([acts(cols, 1000 + t) for t in range(m)])
    y = torch.empty(m, rows, dtype=torch.float32, device="cuda")
    engine.gemm(ty, dev(q), dev(xs), m, y, rows, cols)
    sync()
    want = oracle.matmat(ty, q, rows, cols, xs)
    check_close(y.cpu().numpy(), want, absmag(ty, q, rows, cols, xs))


@pytest.mark.parametrize("m", [4, 8, 16, 64])
def test_gemm_config3(engine, m):
    import torch
    ty, rows, cols = le.Q4_K, 14336, 4096
    q, _ = weights(ty, rows, cols, seed=3)
    xs = np.stack([acts(cols, 2000 + t) for t in range(m)])
    y = torch.empty(m, rows, dtype=torch.float32, device="cuda")
    engine.gemm(ty, dev(q), dev(xs), m, y, rows, cols)
    sync()
    want = oracle.matmat(ty, q, rows, cols, xs)
    check_close(y.cpu().numpy(), want, absmag(ty, q, rows, cols, xs))


@pytest.mark.parametrize("rows,cols,m", [(256, 256, 16), (300, 512, 17), (1000, 1024, 63), (513, 768, 65),
                                          (2048, 2048, 130), (96, 4096, 40)])
def test_gemm_mfma_tiles(engine, rows, cols, m):
    """Ragged token and row tiles of the MFMA GEMM (64 tokens x 256 rows per block)."""
    import torch
    ty = le.Q4_K
    q, _ = weights(ty, rows, cols, seed=rows + m)
    xs = np.stack([acts(cols, 3000 + t) for t in range(m)])
    y = torch.full((m, rows), float("nan"), dtype=torch.float32, device="cuda")
    engine.gemm(ty, dev(q), dev(xs), m, y, rows, cols)
    sync()
    want = oracle.matmat(ty, q, rows, cols, xs)
    check_close(y.cpu().numpy(), want, absmag(ty, q, rows, cols, xs))


def test_gemm_mfma_large_activations(engine):
    """Activations of magnitude ~1e3 exercise the fp16 high/low split away from unit scale."""
    import torch
    ty, rows, cols, m = le.Q4_K, 512, 1024, 32
    q, _ = weights(ty, rows, cols, seed=17)
    xs = np.stack([acts(cols, 4000 + t) * np.float32(1000.0) for t in range(m)])
    y = torch.empty(m, rows, dtype=torch.float32, device="cuda")
    engine.gemm(ty, dev(q), dev(xs), m, y, rows, cols)
    sync()
    want = oracle.matmat(ty, q, rows, cols, xs)
    check_close(y.cpu().numpy(), want, absmag(ty, q, rows, cols, xs))


def test_gemm_workspace_errors(engine):
    import torch
    ty, rows, cols, m = le.Q4_K, 256, 512, 32
    q, _ = weights(ty, rows, cols, seed=2)
    xs = np.stack([acts(cols, 6000 + t) for t in range(m)])
    y = torch.empty(m, rows, dtype=torch.float32, device="cuda")
    small = torch.empty(64, dtype=torch.uint8, device="cuda")
    with pytest.raises(le.LeError) as e:
        engine.gemm(ty, dev(q), dev(xs), m, y, rows, cols, ws=small)
    assert e.value.code == -7
    with pytest.raises(le.LeError) as e:
        engine.gemm(ty, dev(q), dev(xs), m, y, rows, cols, ws=0, ws_bytes=1 << 20)
    assert e.value.code == -1


def test_gemm_config3_m512(engine):
    """Config 3's largest M at its full 14336x4096 shape (the benchmarked launch geometry)."""
    import torch
    ty, rows, cols, m = le.Q4_K, 14336, 4096, 512
    q, _ = weights(ty, rows, cols, seed=3)
    xs = np.stack([acts(cols, 5000 + t) for t in range(m)])
    y = torch.empty(m, rows, dtype=torch.float32, device="cuda")
    engine.gemm(ty, dev(q), dev(xs), m, y, rows, cols)
    sync()
    want = oracle.matmat(ty, q, rows, cols, xs)
    check_close(y.cpu().numpy(), want, absmag(ty, q, rows, cols, xs))


# ------------------------------------------------------------------ edge cases and errors

def test_zero_activation_and_zero_weights(engine):
    import torch
    ty, rows, cols = le.Q4_K, 64, 1024
    q, _ = weights(ty, rows, cols, seed=1)
    y = torch.full((rows,), 7.0, dtype=torch.float32, device="cuda")
    engine.mv(ty, dev(q), dev(np.zeros(cols, np.float32)), y, rows, cols)
    sync()
    assert np.all(y.cpu().numpy() == 0.0)
    zq = np.zeros_like(q)
    engine.mv(ty, dev(zq), dev(acts(cols, 2)), y, rows, cols)
    sync()
    assert np.all(y.cpu().numpy() == 0.0)


def test_error_codes(engine):
    import torch
    x = torch.zeros(1024 + 4, dtype=torch.float32, device="cuda")
    w = torch.zeros(64 * 1024, dtype=torch.uint8, device="cuda")
    y = torch.zeros(64, dtype=torch.float32, device="cuda")
    with pytest.raises(le.LeError) as e:
        engine.mv(99, w, x, y, 8, 1024)
    assert e.value.code == -2
    with pytest.raises(le.LeError) as e:
        engine.mv(le.Q4_K, w, x, y, 8, 1000)
    assert e.value.code == -3
    with pytest.raises(le.LeError) as e:
        engine.mv(le.Q4_K, w, x.data_ptr() + 4, y, 8, 1024)
    assert e.value.code == -4
    with pytest.raises(le.LeError) as e:
        engine.mv(le.Q4_K, w, x, y, 0, 1024)
    assert e.value.code == -3


@pytest.mark.parametrize("path", ["f16", "f16x16", "f16t16", "int8"])
@pytest.mark.parametrize("m", [2, 3, 5, 8, 11, 16])
@pytest.mark.parametrize("rows,cols", [(300, 4096), (64, 2048), (1000, 1024), (4100, 512)])
def test_gemm_few_tokens_staged(fresh_engine, path, m, rows, cols):
    """Few tokens on the staged kernels: the f16 MFMA kernel for 3..8 tokens (tokens as MFMA
    rows, T = 4 or 8; 9..16 tokens under the default gm_mh_max=16 as two 8-token groups streaming
    the same row tiles side by side, or with gm_mh_t16=1 as one 16-token group) and the int8
    multi-token matvec (T = 2, 4 or 8 per pass, option gm_mh=0), with partial token groups (3, 5,
    11), a second group (11, 16 > 8) and ragged row tiles."""
    import torch
    engine = fresh_engine
    engine.set_option("gm_min_m", 64)
    engine.set_option("gm_mh", 0 if path == "int8" else 1)
    engine.set_option("gm_mh_max", 16 if path in ("f16x16", "f16t16") else 8)
    engine.set_option("gm_mh_t16", 1 if path == "f16t16" else 0)
    ty = le.Q4_K
    q, _ = weights(ty, rows, cols, seed=31 + m)
    xs = np.stack([acts(cols, 6000 + 17 * m + t) for t in range(m)])
    y = torch.full((m, rows), float("nan"), dtype=torch.float32, device="cuda")
    engine.gemm(ty, dev(q), dev(xs), m, y, rows, cols)
    sync()
    want = oracle.matmat(ty, q, rows, cols, xs)
    check_close(y.cpu().numpy(), want, absmag(ty, q, rows, cols, xs))


@pytest.mark.parametrize("shape", [14, 18, 24, 22])
@pytest.mark.parametrize("m", [4, 8, 16])
def test_gemm_few_tokens_every_shape(fresh_engine, shape, m):
    """Every (P, waves) shape of the few-token f16 kernel (option gm_mh_shape = 10 P + waves), so a
    wave builds 1 to 8 local super-blocks of activations (the rows loaded before its first weight
    item and, past eight rows, the rows loaded after it), at 4, 8 and 16 (one group) tokens."""
    import torch
    engine = fresh_engine
    engine.set_option("gm_min_m", 64)
    engine.set_option("gm_mh_max", 16)
    engine.set_option("gm_mh_t16", 1)
    engine.set_option("gm_mh_shape", shape)
    ty, rows, cols = le.Q4_K, 200, 4096
    q, _ = weights(ty, rows, cols, seed=41 + shape)
    xs = np.stack([acts(cols, 7000 + 13 * m + t) for t in range(m)])
    y = torch.full((m, rows), float("nan"), dtype=torch.float32, device="cuda")
    engine.gemm(ty, dev(q), dev(xs), m, y, rows, cols)
    sync()
    check_close(y.cpu().numpy(), oracle.matmat(ty, q, rows, cols, xs), absmag(ty, q, rows, cols, xs))


@pytest.mark.parametrize("m", [16, 128])
def test_gemm_activation_split(fresh_engine, m):
    """gm_split=1 carries each activation as two fp16 halves: the result then agrees with the fp64
    oracle to about 2^-22 of sum|w*x| (fp32 accumulation), well inside the single-half bound of
    2^-11 that the default meets."""
    import torch
    engine = fresh_engine
    ty, rows, cols = le.Q4_K, 512, 2048
    q, _ = weights(ty, rows, cols, seed=23)
    xs = np.stack([acts(cols, 5000 + t) for t in range(m)])
    want = oracle.matmat(ty, q, rows, cols, xs)
    mag = absmag(ty, q, rows, cols, xs)
    errs = {}
    for split in (0, 1):
        engine.set_option("gm_split", split)
        y = torch.empty(m, rows, dtype=torch.float32, device="cuda")
        engine.gemm(ty, dev(q), dev(xs), m, y, rows, cols)
        sync()
        errs[split] = float(np.max(np.abs(y.cpu().numpy() - want) / mag))
    assert errs[0] <= 2.0 ** -11, errs
    assert errs[1] <= 1e-5, errs


def test_options_validated(fresh_engine):
    """Every documented launch-policy knob is accepted with a valid value; bad names and values
    are refused with LE_ERR_ARG and leave the context usable."""
    good = {"mv_block": 512, "mv_blocks_per_cu": 1, "mv_shape": 0, "mq": 1, "ms": 1, "mq_waves": 4, "mq_steps": 2,
            "mq_blocks_per_cu": 2, "mq_waves_auto": 1, "ms_p": 2, "ms_p6": 2, "ms_piq": 2, "mq6": 1, "mqiq": 1, "ms_t": 1, "gm_mh": 1, "gm_mh_shape": 0, "gm_mh_max": 16, "gm_min_m": 5,
            "gm_tile": 0, "gm_ksplit": 0, "gm_pc": 1, "gm_split": 0, "moe_mfma": 1, "moe_fused": 1, "moe_fused_min_tok": 3,
            "moe_fast": 1, "gq": 1, "gq_min_m": 9, "gq_cfg": 0, "gq_ksplit": 0}
    engine = fresh_engine
    for k, v in good.items():
        engine.set_option(k, v)
    for k, v in [("no_such_option", 1), ("gm_tile", 33), ("gm_ksplit", 3), ("gm_split", 2), ("gm_mh_shape", 13), ("gm_mh_max", 12), ("ms_p6", 4), ("ms_piq", 3), ("gq_cfg", 13), ("gq_ksplit", 3), ("gq_min_m", 0)]:
        with pytest.raises(le.LeError) as e:
            engine.set_option(k, v)
        assert e.value.code == -1, (k, v)
    # still usable
    import torch
    q, _ = weights(le.Q4_K, 64, 512, seed=3)
    x = acts(512, 4)
    y = torch.empty(64, dtype=torch.float32, device="cuda")
    engine.mv(le.Q4_K, dev(q), dev(x), y, 64, 512)
    sync()
    check_close(y.cpu().numpy(), oracle.matvec(le.Q4_K, q, 64, 512, x), absmag(le.Q4_K, q, 64, 512, x)[0])


@pytest.mark.parametrize("name", ["Q4_K", "Q6_K", "IQ2_XXS", "IQ3_XXS"])
@pytest.mark.parametrize("opts", [{"mq_waves": 8}, {"mq_waves": 2}, {"ms": 0}, {"mq": 0}])
def test_matvec_launch_options(fresh_engine, name, opts):
    """Every staged-kernel shape the options can select exists and gives the same answer."""
    import torch
    engine = fresh_engine
    ty, rows, cols = le.TYPES[name], 300, 4096
    for k, v in opts.items():
        engine.set_option(k, v)
    q, _ = weights(ty, rows, cols, seed=77 + ty)
    x = acts(cols, 78)
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    engine.mv(ty, dev(q), dev(x), y, rows, cols)
    sync()
    check_close(y.cpu().numpy(), oracle.matvec(ty, q, rows, cols, x), absmag(ty, q, rows, cols, x)[0])


@pytest.mark.parametrize("name,opt", [("Q4_K", "ms_p"), ("Q8_0", "ms_p80"), ("IQ2_XXS", "ms_piq")])
@pytest.mark.parametrize("rows,cols", [(64, 8192), (4000, 8192)])
def test_staged_shape_not_instantiated(fresh_engine, name, opt, rows, cols):
    """Four super-blocks per item: with few row tiles the waves double to 8, and (P = 4, 8 waves)
    has no kernel; the launch lowers P to an instantiated shape instead of failing."""
    import torch
    ty = le.TYPES[name]
    fresh_engine.set_option(opt, 4)
    q, _ = weights(ty, rows, cols, seed=rows + ty)
    x = acts(cols, 3 + rows)
    y = torch.full((rows,), float("nan"), device="cuda")
    print("staged shape fallback", name, opt, rows, cols, flush=True)
    fresh_engine.mv(ty, dev(q), dev(x), y, rows, cols)
    sync()
    want = oracle.matvec(ty, q, rows, cols, x)
    check_close(y.cpu().numpy(), want, absmag(ty, q, rows, cols, x)[0])
