"""GPU parity of the wider formats (Q4_0, Q3_K, Q5_K, IQ2_S) and of the int8 activation mode.

Inputs are arbitrary GGUF block bytes with the f16 super-block scales replaced by bounded finite
values (every scale code, grid index and sign pattern occurs), so the kernels see what real GGUF
tensors hold. Bars: dequant bit-exact; le_matvec / le_gemm within the 1e-3 parity bar against the
oracle's cpu_ref::matvec / matmat; quant_x bit-exact against the oracle's quant_x; le_matvec_q8
within 1e-5 * sum|w * xa| of the oracle's udot-based matvec (the integer dots are exact on both
sides, only the fp32 summation order differs)."""
import numpy as np
import pytest

import lastengine_amd as le
import oracle
from tests.util import acts, check_close, random_blocks

pytestmark = pytest.mark.gpu

NEW = ["Q4_0", "Q3_K", "Q5_K", "IQ2_S"]
ALL = list(le.MV_TYPES)


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def sync():
    import torch
    torch.cuda.synchronize()


@pytest.mark.parametrize("name", NEW)
@pytest.mark.parametrize("rows,cols", [(8, 1024), (37, 768), (3, 4096)])
def test_new_dequant_bit_exact(engine, name, rows, cols):
    import torch
    ty = le.MV_TYPES[name]
    q = random_blocks(ty, rows, cols, seed=rows * 7 + cols + ty)
    out = torch.empty(rows, cols, dtype=torch.float32, device="cuda")
    engine.dequant_rows(ty, dev(q), out, rows, cols)
    sync()
    want = oracle.dequant_rows(ty, q, rows, cols)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("name", NEW)
def test_new_dequant_raw_bytes(engine, name):
    """Unbounded bytes (subnormal, Inf and NaN scales): non-NaN values bit-identical, NaN where NaN."""
    import torch
    ty = le.MV_TYPES[name]
    rows, cols = 16, 1024
    q = np.random.default_rng(ty + 1).integers(0, 256, size=(rows, le.row_bytes(ty, cols)), dtype=np.uint8)
    out = torch.empty(rows, cols, dtype=torch.float32, device="cuda")
    engine.dequant_rows(ty, dev(q), out, rows, cols)
    sync()
    want = oracle.dequant_rows(ty, q, rows, cols)
    got = out.cpu().numpy()
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def _absmag(ty, q, rows, cols, xs):
    w = oracle.dequant_rows(ty, q, rows, cols).astype(np.float64)
    return np.abs(np.atleast_2d(xs).astype(np.float64)) @ np.abs(w).T


@pytest.mark.parametrize("name", NEW)
@pytest.mark.parametrize("rows,cols", [(64, 256), (333, 4096), (77, 768), (40, 14336), (1, 512)])
def test_new_matvec_parity(engine, name, rows, cols):
    import torch
    ty = le.MV_TYPES[name]
    q = random_blocks(ty, rows, cols, seed=ty * 31 + rows)
    x = acts(cols, 5 + rows)
    y = torch.full((rows,), float("nan"), device="cuda")
    engine.mv(ty, dev(q), dev(x), y, rows, cols)
    sync()
    want = oracle.matvec(ty, q, rows, cols, x)
    check_close(y.cpu().numpy(), want, _absmag(ty, q, rows, cols, x)[0])


@pytest.mark.parametrize("name", NEW)
@pytest.mark.parametrize("m", [2, 5, 17])
def test_new_gemm_parity(engine, name, m):
    import torch
    ty = le.MV_TYPES[name]
    rows, cols = 96, 2048
    q = random_blocks(ty, rows, cols, seed=ty + m)
    xs = np.stack([acts(cols, 50 + t) for t in range(m)])
    assert engine.gemm_workspace_size(ty, m, cols) > 0  # the matrix-core GEMM's activation fragments
    y = torch.full((m * rows,), float("nan"), device="cuda")
    engine.gemm(ty, dev(q), dev(xs), m, y, rows, cols)
    sync()
    want = oracle.matmat(ty, q, rows, cols, xs)
    check_close(y.cpu().numpy().reshape(m, rows), want, _absmag(ty, q, rows, cols, xs))


def test_unknown_type_rejected_by_moe(engine):
    import torch
    with pytest.raises(le.LeError) as e:
        engine.moe(7, 7, le.Q6_K, dev(np.zeros(16, np.uint8)), dev(np.zeros(16, np.uint8)),
                   dev(np.zeros(16, np.uint8)), 4, 2, 256, 256, dev(np.zeros(4, np.float32)),
                   dev(np.zeros(256, np.float32)), 1, torch.empty(256, device="cuda"), ws=torch.empty(1 << 20, dtype=torch.uint8, device="cuda"))
    assert e.value.code == -2


# ------------------------------------------------------------------ int8 activation mode

@pytest.mark.parametrize("n", [32, 4096, 14336])
def test_quant_x_bit_exact(engine, n):
    import torch
    x = acts(n, n)
    x[:32] = 0.0            # an all-zero unit
    x[32:64] *= 1e-30
    xq = torch.empty(n, dtype=torch.int8, device="cuda")
    xd = torch.empty(n // 32, dtype=torch.float32, device="cuda")
    xs = torch.empty(n // 32, dtype=torch.int32, device="cuda")
    engine.quant_x(dev(x), xq, xd, xs, n // 32)
    sync()
    wq, wd, ws = oracle.quant_x(x)
    assert np.array_equal(xq.cpu().numpy(), wq)
    assert np.array_equal(xd.cpu().numpy().view(np.uint32), wd.view(np.uint32))
    assert np.array_equal(xs.cpu().numpy(), ws)


@pytest.mark.parametrize("name", ALL)
@pytest.mark.parametrize("rows,cols", [(100, 4096), (40, 14336), (77, 768)])
def test_matvec_q8_parity(engine, name, rows, cols):
    import torch
    ty = le.MV_TYPES[name]
    q = random_blocks(ty, rows, cols, seed=ty * 3 + cols)
    x = acts(cols, 9 + rows)
    xq, xd, xs = oracle.quant_x(x)
    y = torch.full((rows,), float("nan"), device="cuda")
    engine.mv_q8(ty, None, dev(xq), dev(xd), dev(xs), y, rows, cols, 0, 1, w=dev(q))
    sync()
    want = oracle.matvec_q8(ty, q, rows, cols, xq, xd, xs)
    wd = oracle.dequant_rows(ty, q, rows, cols).astype(np.float64)
    xa = np.repeat(xd.astype(np.float64), 32) * xq.astype(np.float64)
    mag = np.abs(wd) @ np.abs(xa)
    got = y.cpu().numpy()
    assert np.all(np.isfinite(got))
    assert np.all(np.abs(got - want) <= 1e-5 * mag + 1e-30), float(np.max(np.abs(got - want) / mag))


def test_matvec_q8_slots_and_pointer_table(engine):
    """Two slots through a device pointer table with per-slot activations (xstride = cols), the
    reference's fused gate+up launch shape with distinct inputs."""
    import torch
    ty, rows, cols = le.Q4_K, 48, 2048
    qs = [random_blocks(ty, rows, cols, seed=100 + s) for s in range(2)]
    xs_ = [acts(cols, 200 + s) for s in range(2)]
    quant = [oracle.quant_x(x) for x in xs_]
    dws = [dev(q) for q in qs]
    ptrs = dev(np.array([w.data_ptr() for w in dws], dtype=np.uint64))
    xq = dev(np.concatenate([t[0] for t in quant]))
    xd = dev(np.concatenate([t[1] for t in quant]))
    xsum = dev(np.concatenate([t[2] for t in quant]))
    y = torch.full((2 * rows,), float("nan"), device="cuda")
    engine.mv_q8(ty, ptrs, xq, xd, xsum, y, rows, cols, cols, 2)
    sync()
    got = y.cpu().numpy().reshape(2, rows)
    for s in range(2):
        want = oracle.matvec_q8(ty, qs[s], rows, cols, *quant[s])
        np.testing.assert_allclose(got[s], want, rtol=1e-4, atol=1e-6 * np.abs(want).max())


@pytest.mark.parametrize("n", [32, 4096, 14336])
def test_rms_quant(engine, n):
    """le_rms_quant: o within a few ulp of cpu_ref::rms (the sum of squares is reduced in another
    order), and xq/xd/xs bit-identical to quant_x of that o."""
    import torch
    x = acts(n, 3 * n)
    w = acts(n, 3 * n + 1)
    o = torch.empty(n, dtype=torch.float32, device="cuda")
    xq = torch.empty(n, dtype=torch.int8, device="cuda")
    xd = torch.empty(n // 32, dtype=torch.float32, device="cuda")
    xs = torch.empty(n // 32, dtype=torch.int32, device="cuda")
    engine.rms_quant(dev(x), dev(w), o, xq, xd, xs, n, 1e-6)
    sync()
    og = o.cpu().numpy()
    want = oracle.rms(x, w, 1e-6)
    np.testing.assert_allclose(og, want, rtol=4e-6, atol=1e-7 * np.abs(want).max())
    wq, wd, ws = oracle.quant_x(og)
    assert np.array_equal(xq.cpu().numpy(), wq)
    assert np.array_equal(xd.cpu().numpy().view(np.uint32), wd.view(np.uint32))
    assert np.array_equal(xs.cpu().numpy(), ws)


SWIGLU_SHAPES = [("Q6_K", 4096, 14336), ("Q4_K", 4096, 14336), ("Q4_K", 333, 1024), ("Q8_0", 200, 4096),
                 ("IQ2_XXS", 64, 4096), ("IQ3_XXS", 96, 2048), ("Q4_0", 100, 768), ("Q3_K", 64, 2048),
                 ("Q5_K", 77, 4096), ("IQ2_S", 50, 1024)]


@pytest.mark.parametrize("name,rows,cols", SWIGLU_SHAPES)
def test_matvec_swiglu(engine, name, rows, cols):
    """le_matvec_swiglu against cpu_ref: down . (silu(gate) * up) from one gate | up vector (the
    Q6_K 4096x14336 case is config 2's down projection on the staged matrix-core kernel)."""
    import torch
    ty = le.MV_TYPES[name]
    q = random_blocks(ty, rows, cols, seed=ty + rows + cols)
    gu = acts(2 * cols, 31 + cols)
    y = torch.full((rows,), float("nan"), device="cuda")
    engine.mv_swiglu(ty, dev(q), dev(gu), y, rows, cols)
    sync()
    a = oracle.swiglu(gu[:cols], gu[cols:])
    want = oracle.matvec(ty, q, rows, cols, a)
    check_close(y.cpu().numpy(), want, _absmag(ty, q, rows, cols, a)[0])


def test_matvec_swiglu_slots(engine):
    """Two slots through a pointer table, each with its own gate | up vector (xstride = 2 cols)."""
    import torch
    ty, rows, cols = le.Q6_K, 256, 768
    qs = [random_blocks(ty, rows, cols, seed=900 + s) for s in range(2)]
    gus = [acts(2 * cols, 910 + s) for s in range(2)]
    dws = [dev(q) for q in qs]
    ptrs = dev(np.array([w.data_ptr() for w in dws], dtype=np.uint64))
    y = torch.full((2 * rows,), float("nan"), device="cuda")
    engine.mv_swiglu(ty, None, dev(np.concatenate(gus)), y, rows, cols, ptrs=ptrs, xstride=2 * cols, slots=2)
    sync()
    got = y.cpu().numpy().reshape(2, rows)
    for s in range(2):
        a = oracle.swiglu(gus[s][:cols], gus[s][cols:])
        check_close(got[s], oracle.matvec(ty, qs[s], rows, cols, a), _absmag(ty, qs[s], rows, cols, a)[0])


@pytest.mark.parametrize("name", ["Q4_K", "Q6_K", "IQ3_XXS"])
def test_matvec_q8_vector_path(fresh_engine, name):
    """The int8 mode runs on the staged matrix-core kernels for these types by default; option
    mq_q8=0 keeps them on the vector kernels. Both meet the same bar against the oracle."""
    import torch
    ty = le.MV_TYPES[name]
    rows, cols = 96, 4096
    q = random_blocks(ty, rows, cols, seed=ty + 5)
    x = acts(cols, 17)
    xq, xd, xs = oracle.quant_x(x)
    want = oracle.matvec_q8(ty, q, rows, cols, xq, xd, xs)
    wd = oracle.dequant_rows(ty, q, rows, cols).astype(np.float64)
    mag = np.abs(wd) @ np.abs(np.repeat(xd.astype(np.float64), 32) * xq.astype(np.float64))
    for flag in (1, 0):
        fresh_engine.set_option("mq_q8", flag)
        y = torch.full((rows,), float("nan"), device="cuda")
        fresh_engine.mv_q8(ty, None, dev(xq), dev(xd), dev(xs), y, rows, cols, 0, 1, w=dev(q))
        sync()
        got = y.cpu().numpy()
        assert np.all(np.abs(got - want) <= 1e-5 * mag + 1e-30), (flag, float(np.max(np.abs(got - want) / mag)))


@pytest.mark.parametrize("name,opt", [("Q8_0", "ms80"), ("Q4_0", "ms40"), ("Q5_K", "ms5k"), ("Q3_K", "ms3k"), ("IQ2_S", "ms2s")])
@pytest.mark.parametrize("rows,cols", [(333, 4096), (40, 14336), (17, 256), (64, 768)])
def test_matvec_staged_q8_0_q4_0(fresh_engine, name, opt, rows, cols):
    """Q8_0, Q4_0, Q5_K, Q3_K and IQ2_S batch-1 matvec on the staged matrix-core kernels (option 1) and on the vector
    kernels (option 0): both meet the parity bar against the oracle, with and without the int8
    activation mode."""
    import torch
    ty = le.MV_TYPES[name]
    q = random_blocks(ty, rows, cols, seed=ty * 13 + rows + cols)
    x = acts(cols, 3 + rows)
    want = oracle.matvec(ty, q, rows, cols, x)
    mag = _absmag(ty, q, rows, cols, x)[0]
    xq, xd, xs = oracle.quant_x(x)
    want8 = oracle.matvec_q8(ty, q, rows, cols, xq, xd, xs)
    wd = oracle.dequant_rows(ty, q, rows, cols).astype(np.float64)
    mag8 = np.abs(wd) @ np.abs(np.repeat(xd.astype(np.float64), 32) * xq.astype(np.float64))
    for flag in (1, 0):
        fresh_engine.set_option(opt, flag)
        print("staged", name, flag, rows, cols, flush=True)
        y = torch.full((rows,), float("nan"), device="cuda")
        fresh_engine.mv(ty, dev(q), dev(x), y, rows, cols)
        sync()
        check_close(y.cpu().numpy(), want, mag)
        y = torch.full((rows,), float("nan"), device="cuda")
        fresh_engine.mv_q8(ty, None, dev(xq), dev(xd), dev(xs), y, rows, cols, 0, 1, w=dev(q))
        sync()
        got = y.cpu().numpy()
        assert np.all(np.abs(got - want8) <= 1e-5 * mag8 + 1e-30), (flag, float(np.max(np.abs(got - want8) / mag8)))
