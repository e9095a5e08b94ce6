"""GPU parity of the grouped matmul (le_mm_grouped, the reference's mm_impl over off / in_idx /
out_idx, src/cuda/kernels.cu:679-719) and of the MoE layer over per-expert pointer tables
(build_ptrs' layout, src/cuda/kernels.cu:458-468), against the oracle."""
import numpy as np
import pytest

import lastengine_amd as le
import oracle
from tests.util import weights, acts, check_close, wbytes

pytestmark = pytest.mark.gpu


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def grouping(counts, n_src, seed):
    """off / in_idx / out_idx for slots with the given pair counts: sources drawn at random, output
    rows a random permutation of the pairs."""
    rng = np.random.default_rng(seed)
    off = np.zeros(len(counts) + 1, dtype=np.int32)
    off[1:] = np.cumsum(counts)
    npair = int(off[-1])
    in_idx = rng.integers(0, n_src, size=npair).astype(np.int32)
    out_idx = rng.permutation(npair).astype(np.int32)
    return off, in_idx, out_idx


@pytest.mark.parametrize("name", list(le.MV_TYPES))
@pytest.mark.parametrize("counts", [(0, 5, 300, 17, 1, 128, 64, 40), (20, 40, 33, 60), (3, 3, 3)])
@pytest.mark.parametrize("tables", [False, True])
def test_mm_grouped(engine, name, counts, tables):
    import torch
    ty = le.MV_TYPES[name]
    nslot, rows, cols, n_src = len(counts), 320, 1024, 200
    print("mm_grouped", name, counts, tables, flush=True)
    q = wbytes(ty, nslot * rows, cols, seed=60 + ty)
    xs = np.stack([acts(cols, 7700 + t) for t in range(n_src)])
    off, in_idx, out_idx = grouping(counts, n_src, seed=ty + len(counts))
    npair = int(off[-1])
    dq = dev(q)
    ptrs = None
    if tables:  # slot s's rows anywhere in memory: here the slabs in reverse order
        rb = le.row_bytes(ty, cols) * rows
        order = list(reversed(range(nslot)))
        arena = torch.cat([dq.reshape(nslot, -1)[s] for s in order])
        base = arena.data_ptr()
        ptrs = dev(np.array([base + order.index(s) * rb for s in range(nslot)], dtype=np.uint64))
        w = None
    else:
        w = dq
    y = torch.full((npair, rows), float("nan"), dtype=torch.float32, device="cuda")
    engine.mm_grouped(ty, dev(off), dev(in_idx), dev(out_idx), nslot, npair, dev(xs), y, rows, cols, ptrs=ptrs, w=w)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    rbs = le.row_bytes(ty, cols) * rows
    for s in range(nslot):
        lo, hi = off[s], off[s + 1]
        if hi == lo:
            continue
        slab = q.reshape(-1)[s * rbs:(s + 1) * rbs]
        xsel = xs[in_idx[lo:hi]]
        want = oracle.matmat(ty, slab, rows, cols, xsel)
        wf = oracle.dequant_rows(ty, slab, rows, cols).astype(np.float64)
        mag = np.abs(xsel.astype(np.float64)) @ np.abs(wf).T
        check_close(got[out_idx[lo:hi]], want, mag)


@pytest.mark.parametrize("n_tok", [1, 4, 8, 20, 100])
def test_moe_pointer_tables(engine, n_tok):
    """le_moe_layer_ptrs gives the same bits as le_moe_layer on the same experts (here placed in a
    shuffled arena): only the weight addressing differs."""
    import torch
    tg, td, n_exp, k, hidden, ff = le.Q4_K, le.Q6_K, 16, 4, 2048, 768
    g, _ = weights(tg, n_exp * ff, hidden, 800)
    u, _ = weights(tg, n_exp * ff, hidden, 801)
    d, _ = weights(td, n_exp * hidden, ff, 802)
    h = acts(n_tok * hidden, 803).reshape(n_tok, hidden)
    lg = acts(n_tok * n_exp, 804).reshape(n_tok, n_exp)
    dg, du, dd, dh, dl = dev(g), dev(u), dev(d), dev(h), dev(lg)
    rng = np.random.default_rng(n_tok)

    def table(t, nrows, ty, ncols):
        eb = nrows * le.row_bytes(ty, ncols)
        perm = rng.permutation(n_exp)
        arena = torch.cat([t.reshape(n_exp, -1)[e] for e in perm])
        pos = np.argsort(perm)
        return arena, dev(np.array([arena.data_ptr() + int(pos[e]) * eb for e in range(n_exp)], dtype=np.uint64))

    ag, pg = table(dg, ff, tg, hidden)
    au, pu = table(du, ff, tg, hidden)
    ad, pd = table(dd, hidden, td, ff)
    out1 = torch.empty(n_tok, hidden, dtype=torch.float32, device="cuda")
    out2 = torch.empty(n_tok, hidden, dtype=torch.float32, device="cuda")
    engine.moe(tg, tg, td, dg, du, dd, n_exp, k, hidden, ff, dl, dh, n_tok, out1)
    engine.moe_ptrs(tg, tg, td, pg, pu, pd, n_exp, k, hidden, ff, dl, dh, n_tok, out2)
    torch.cuda.synchronize()
    a, b = out1.cpu().numpy(), out2.cpu().numpy()
    assert np.all(np.isfinite(a))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("name", ["Q4_K", "Q6_K"])
def test_mm_grouped_many_slots(engine, name):
    """More slots than one round of the blocks' slot walk (256 per round): pairs only in a few
    slots on both sides of the round and wave boundaries (63/64, 255/256), one slot spanning two
    32-pair tiles, the rest empty."""
    import torch
    ty = le.MV_TYPES[name]
    nslot, rows, cols, n_src = 300, 128, 512, 64
    counts = [0] * nslot
    for s, c in ((0, 3), (63, 1), (64, 9), (255, 2), (256, 40), (257, 1), (299, 5)):
        counts[s] = c
    print("mm_grouped many slots", name, flush=True)
    q = wbytes(ty, nslot * rows, cols, seed=90 + ty)
    xs = np.stack([acts(cols, 8800 + t) for t in range(n_src)])
    off, in_idx, out_idx = grouping(counts, n_src, seed=ty)
    npair = int(off[-1])
    y = torch.full((npair, rows), float("nan"), dtype=torch.float32, device="cuda")
    engine.mm_grouped(ty, dev(off), dev(in_idx), dev(out_idx), nslot, npair, dev(xs), y, rows, cols, w=dev(q))
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    rbs = le.row_bytes(ty, cols) * rows
    for s in range(nslot):
        lo, hi = off[s], off[s + 1]
        if hi == lo:
            continue
        slab = q.reshape(-1)[s * rbs:(s + 1) * rbs]
        xsel = xs[in_idx[lo:hi]]
        want = oracle.matmat(ty, slab, rows, cols, xsel)
        wf = oracle.dequant_rows(ty, slab, rows, cols).astype(np.float64)
        mag = np.abs(xsel.astype(np.float64)) @ np.abs(wf).T
        check_close(got[out_idx[lo:hi]], want, mag)


@pytest.mark.parametrize("name", ["Q4_K", "Q6_K", "Q8_0", "IQ2_XXS", "Q5_K"])
@pytest.mark.parametrize("cols", [1024, 4096])
def test_mm_grouped_prepass_forms(engine, name, cols):
    """The activation pre-pass run one wave per pair (K <= 4096) and one block per pair give the
    same bits: both take the row's max magnitude and convert every value the same way."""
    import torch
    ty = le.MV_TYPES[name]
    counts = (0, 37, 200, 5, 64, 1)
    nslot, rows, n_src = len(counts), 128, 90
    print("mm_grouped prepass forms", name, cols, flush=True)
    dq = dev(wbytes(ty, nslot * rows, cols, seed=80 + ty))
    xs = dev(np.stack([acts(cols, 8100 + t) for t in range(n_src)]))
    off, in_idx, out_idx = grouping(counts, n_src, seed=ty)
    npair = int(off[-1])
    outs = []
    try:
        for xw in (1, 0):
            engine.set_option("mmg_xw", xw)
            y = torch.full((npair, rows), float("nan"), dtype=torch.float32, device="cuda")
            engine.mm_grouped(ty, dev(off), dev(in_idx), dev(out_idx), nslot, npair, xs, y, rows, cols, w=dq)
            torch.cuda.synchronize()
            outs.append(y.cpu().numpy())
    finally:
        engine.set_option("mmg_xw", 1)
    assert np.isfinite(outs[0]).all()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


@pytest.mark.parametrize("name", ["Q6_K", "Q8_0", "Q4_0"])
def test_mm_grouped_four_wave_tiles(engine, name):
    """Sparse slots (32-pair tiles) of the types whose 8-wave block fills half the LDS run on 4-wave
    32 x 128 blocks; both give the same bits (a pair's sum runs over K in the same order)."""
    import torch
    ty = le.MV_TYPES[name]
    counts = (3, 0, 17, 1, 40, 2, 9)
    nslot, rows, cols, n_src = len(counts), 320, 768, 60
    q = wbytes(ty, nslot * rows, cols, seed=95 + ty)
    xs_h = np.stack([acts(cols, 8500 + t) for t in range(n_src)])
    off, in_idx, out_idx = grouping(counts, n_src, seed=ty + 5)
    npair = int(off[-1])
    dq, xs = dev(q), dev(xs_h)
    outs = []
    try:
        for w4 in (1, 0):
            engine.set_option("mmg_w4", w4)
            y = torch.full((npair, rows), float("nan"), dtype=torch.float32, device="cuda")
            engine.mm_grouped(ty, dev(off), dev(in_idx), dev(out_idx), nslot, npair, xs, y, rows, cols, w=dq)
            torch.cuda.synchronize()
            outs.append(y.cpu().numpy())
    finally:
        engine.set_option("mmg_w4", 1)
    assert np.isfinite(outs[0]).all()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    rbs = le.row_bytes(ty, cols) * rows
    for s in (2, 4):
        lo, hi = off[s], off[s + 1]
        slab = q.reshape(-1)[s * rbs:(s + 1) * rbs]
        xsel = xs_h[in_idx[lo:hi]]
        want = oracle.matmat(ty, slab, rows, cols, xsel)
        wf = oracle.dequant_rows(ty, slab, rows, cols).astype(np.float64)
        check_close(outs[0][out_idx[lo:hi]], want, np.abs(xsel.astype(np.float64)) @ np.abs(wf).T)
