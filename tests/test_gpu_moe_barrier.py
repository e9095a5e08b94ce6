"""The one-launch MoE layer's device-wide barrier (5..8 tokens at hidden 2048): a forced give-up is
reported (NaN outputs, le_moe_check -> LE_ERR_TIMEOUT) and leaves nothing behind that breaks the
next call; launches on different workspaces keep separate barrier state. The give-up is forced
from the host with a zero spin limit, so every kernel still exits normally."""
import numpy as np
import pytest

import lastengine_amd as le
from tests.test_gpu_moe import dev, reference
from tests.util import weights, acts, check_close

pytestmark = pytest.mark.gpu

TG, TD, N_EXP, K, HIDDEN, FF = le.Q4_K, le.Q6_K, 16, 4, 2048, 768


def inputs(n_tok, seed):
    g, _ = weights(TG, N_EXP * FF, HIDDEN, seed)
    u, _ = weights(TG, N_EXP * FF, HIDDEN, seed + 1)
    d, _ = weights(TD, N_EXP * HIDDEN, FF, seed + 2)
    h = acts(n_tok * HIDDEN, seed + 3).reshape(n_tok, HIDDEN)
    lg = acts(n_tok * N_EXP, seed + 4).reshape(n_tok, N_EXP)
    return g, u, d, h, lg


def call(engine, g, u, d, h, lg, ws):
    import torch
    n_tok = h.shape[0]
    out = torch.full((n_tok, HIDDEN), 7.0, dtype=torch.float32, device="cuda")
    engine.moe(TG, TG, TD, g, u, d, N_EXP, K, HIDDEN, FF, lg, h, n_tok, out, ws=ws)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_barrier_give_up_then_recover(fresh_engine):
    import torch
    engine = fresh_engine
    n_tok = 5
    g, u, d, h, lg = inputs(n_tok, 500)
    dg, du, dd, dh, dl = dev(g), dev(u), dev(d), dev(h), dev(lg)
    ws = torch.empty(engine.moe_workspace_size(n_tok, K, FF), dtype=torch.uint8, device="cuda")
    engine.moe_check(ws)  # an uninitialised workspace reports no failure
    engine.set_option("moe_spin_limit", 0)  # the barrier gives up at once
    print("moe barrier: forced give-up", flush=True)
    bad = call(engine, dg, du, dd, dh, dl, ws)
    assert np.all(np.isnan(bad)), "a launch whose barrier gave up must write NaN everywhere"
    with pytest.raises(le.LeError) as e:
        engine.moe_check(ws)
    assert e.value.code == -8
    engine.moe_check(ws)  # the check cleared the status
    engine.set_option("moe_spin_limit", 1 << 20)
    print("moe barrier: recovery call", flush=True)
    got = call(engine, dg, du, dd, dh, dl, ws)
    engine.moe_check(ws)
    want, _, _, mag = reference(TG, TD, g, u, d, N_EXP, K, HIDDEN, FF, h, lg)
    check_close(got, want, mag)


def test_barrier_separate_workspaces(fresh_engine):
    """Alternating launches on two workspaces (and token counts) stay correct: each workspace's
    flags hold only its own launches' epochs."""
    import torch
    engine = fresh_engine
    cases = []
    for n_tok, seed in ((5, 600), (8, 610)):
        g, u, d, h, lg = inputs(n_tok, seed)
        ws = torch.empty(engine.moe_workspace_size(n_tok, K, FF), dtype=torch.uint8, device="cuda")
        want, _, _, mag = reference(TG, TD, g, u, d, N_EXP, K, HIDDEN, FF, h, lg)
        cases.append(((dev(g), dev(u), dev(d), dev(h), dev(lg)), ws, want, mag))
    for rep in range(3):
        for (args, ws, want, mag) in cases:
            print("moe barrier: workspace alternation", rep, flush=True)
            got = call(engine, *args, ws)
            check_close(got, want, mag)
            engine.moe_check(ws)


def test_barrier_graph_replays(fresh_engine):
    """One captured one-launch layer (the only launch on its workspace), replayed with new token
    activations copied in between: each replay's launch takes a fresh epoch from the workspace,
    so its barrier waits for this replay's gate/up images (an epoch fixed in the kernel arguments
    would let the second replay's barrier pass at once and read the previous replay's images)."""
    import torch
    engine = fresh_engine
    n_tok = 5
    g, u, d, h0, lg = inputs(n_tok, 700)
    dg, du, dd, dl = dev(g), dev(u), dev(d), dev(lg)
    dh = dev(h0)
    ws = torch.zeros(engine.moe_workspace_size(n_tok, K, FF), dtype=torch.uint8, device="cuda")
    out = torch.empty(n_tok, HIDDEN, dtype=torch.float32, device="cuda")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        engine.moe(TG, TG, TD, dg, du, dd, N_EXP, K, HIDDEN, FF, dl, dh, n_tok, out, ws=ws, stream=s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        engine.moe(TG, TG, TD, dg, du, dd, N_EXP, K, HIDDEN, FF, dl, dh, n_tok, out, ws=ws, stream=s)
    torch.cuda.synchronize()
    for rep in range(4):
        h = acts(n_tok * HIDDEN, 710 + rep).reshape(n_tok, HIDDEN)
        dh.copy_(torch.from_numpy(h))  # eager work between the replays
        out.fill_(7.0)
        torch.cuda.synchronize()
        print("moe barrier: graph replay", rep, flush=True)
        graph.replay()
        torch.cuda.synchronize()
        engine.moe_check(ws)
        want, _, _, mag = reference(TG, TD, g, u, d, N_EXP, K, HIDDEN, FF, h, lg)
        check_close(out.cpu().numpy(), want, mag)
