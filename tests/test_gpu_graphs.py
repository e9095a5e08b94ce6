"""Captured HIP graphs of the product entries, replayed several times with new inputs copied in
between by eager work: every replay must match the oracle (no state carried from the capture or
from the previous replay). Covers the grouped MoE form (routing, grouping and the grouped matmuls
that find their tiles on the device), the K-sliced GEMM with its ordered slice sum, and the decode
matvec."""
import numpy as np
import pytest

import lastengine_amd as le
import oracle
from tests.test_gpu_moe import dev, reference
from tests.util import weights, acts, check_close, wbytes

pytestmark = pytest.mark.gpu


def capture(fn):
    import torch
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        fn(s)  # warm-up on the capture stream (code objects loaded, occupancy queried)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        fn(s)
    torch.cuda.synchronize()
    return graph


@pytest.mark.parametrize("n_tok", [16, 40])
def test_graph_moe_grouped(engine, n_tok):
    import torch
    tg, td, n_exp, k, hidden, ff = le.Q4_K, le.Q6_K, 32, 4, 1024, 512
    g, _ = weights(tg, n_exp * ff, hidden, 900)
    u, _ = weights(tg, n_exp * ff, hidden, 901)
    d, _ = weights(td, n_exp * hidden, ff, 902)
    dg, du, dd = dev(g), dev(u), dev(d)
    dh = torch.zeros(n_tok, hidden, dtype=torch.float32, device="cuda")
    dl = torch.zeros(n_tok, n_exp, dtype=torch.float32, device="cuda")
    out = torch.empty(n_tok, hidden, dtype=torch.float32, device="cuda")
    nws = max(engine.moe_workspace_size(n_tok, k, ff), engine.moe_prefill_workspace_size(n_tok, k, n_exp, hidden, ff))
    ws = torch.zeros(nws, dtype=torch.uint8, device="cuda")
    graph = capture(lambda s: engine.moe(tg, tg, td, dg, du, dd, n_exp, k, hidden, ff, dl, dh, n_tok, out, ws=ws, stream=s))
    for rep in range(4):  # new activations and new routing each time
        h = acts(n_tok * hidden, 910 + rep).reshape(n_tok, hidden)
        lg = acts(n_tok * n_exp, 920 + rep).reshape(n_tok, n_exp)
        dh.copy_(torch.from_numpy(h))
        dl.copy_(torch.from_numpy(lg))
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        print("graph moe grouped", n_tok, "replay", rep, flush=True)
        graph.replay()
        torch.cuda.synchronize()
        want, _, _, mag = reference(tg, td, g, u, d, n_exp, k, hidden, ff, h, lg)
        check_close(out.cpu().numpy(), want, mag)


@pytest.mark.parametrize("name,m", [("Q4_K", 64), ("Q6_K", 40)])
def test_graph_gemm_k_slices(engine, name, m):
    import torch
    ty = le.MV_TYPES[name]
    rows, cols = 1024, 4096
    q = wbytes(ty, rows, cols, seed=930 + ty)
    dq = dev(q)
    x = torch.zeros(m, cols, dtype=torch.float32, device="cuda")
    y = torch.empty(m, rows, dtype=torch.float32, device="cuda")
    ws = torch.zeros(engine.gemm_workspace_size_rows(ty, m, rows, cols), dtype=torch.uint8, device="cuda")
    graph = capture(lambda s: engine.gemm(ty, dq, x, m, y, rows, cols, ws=ws, stream=s))
    wf = oracle.dequant_rows(ty, q, rows, cols).astype(np.float64)
    for rep in range(4):
        xs = np.stack([acts(cols, 940 + 10 * rep + t) for t in range(m)])
        x.copy_(torch.from_numpy(xs))
        y.fill_(float("nan"))
        torch.cuda.synchronize()
        print("graph gemm", name, m, "replay", rep, flush=True)
        graph.replay()
        torch.cuda.synchronize()
        want = oracle.matmat(ty, q, rows, cols, xs)
        mag = np.abs(xs.astype(np.float64)) @ np.abs(wf).T
        check_close(y.cpu().numpy(), want, mag)


def test_graph_matvec(engine):
    import torch
    ty, rows, cols = le.Q4_K, 4096, 4096
    q = wbytes(ty, rows, cols, seed=950)
    dq = dev(q)
    x = torch.zeros(cols, dtype=torch.float32, device="cuda")
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    graph = capture(lambda s: engine.mv(ty, dq, x, y, rows, cols, stream=s))
    wf = oracle.dequant_rows(ty, q, rows, cols).astype(np.float64)
    for rep in range(4):
        xv = acts(cols, 960 + rep)
        x.copy_(torch.from_numpy(xv))
        y.fill_(float("nan"))
        torch.cuda.synchronize()
        print("graph matvec replay", rep, flush=True)
        graph.replay()
        torch.cuda.synchronize()
        want = oracle.matvec(ty, q, rows, cols, xv)
        check_close(y.cpu().numpy()[None, :], want[None, :], (np.abs(wf) @ np.abs(xv.astype(np.float64)))[None, :])
