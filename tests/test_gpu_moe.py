"""GPU parity of the routed MoE layer against the oracle's cpu_ref::moe restatement."""
import numpy as np
import pytest

import lastengine_amd as le
import oracle
from tests.util import weights, acts, check_close, random_blocks, wbytes

pytestmark = pytest.mark.gpu


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def reference(tg, td, g, u, d, n_exp, k, hidden, ff, h, lg):
    """Oracle output plus the condition number sum_s w_s * sum_c |down[r,c] * a_c| per output
    (computed per expert over all the pairs routed to it, from the dequantized weights)."""
    out, idx, w = oracle.moe(tg, tg, td, g, u, d, n_exp, k, hidden, ff, h, lg)
    rbg, rbd = le.row_bytes(tg, hidden), le.row_bytes(td, ff)
    mag = np.zeros_like(out, dtype=np.float64)
    gf, uf, df = g.reshape(-1), u.reshape(-1), d.reshape(-1)
    for e in np.unique(idx):
        ts, ss = np.nonzero(idx == e)
        gw = oracle.dequant_rows(tg, gf[e * ff * rbg:(e + 1) * ff * rbg], ff, hidden).astype(np.float64)
        uw = oracle.dequant_rows(tg, uf[e * ff * rbg:(e + 1) * ff * rbg], ff, hidden).astype(np.float64)
        dw = oracle.dequant_rows(td, df[e * hidden * rbd:(e + 1) * hidden * rbd], hidden, ff).astype(np.float64)
        hh = h[ts].astype(np.float64)
        gg, uu = hh @ gw.T, hh @ uw.T
        a = gg / (1 + np.exp(-gg)) * uu
        mag[ts] += w[ts, ss][:, None] * (np.abs(a) @ np.abs(dw).T)
    return out, idx, w, mag


def run(engine, tg, td, n_exp, k, hidden, ff, n_tok, seed, lg=None, rand=False, ws=None):
    import torch
    if rand:
        g = random_blocks(tg, n_exp * ff, hidden, seed)
        u = random_blocks(tg, n_exp * ff, hidden, seed + 1)
        d = random_blocks(td, n_exp * hidden, ff, seed + 2)
    else:
        g = wbytes(tg, n_exp * ff, hidden, seed)
        u = wbytes(tg, n_exp * ff, hidden, seed + 1)
        d = wbytes(td, n_exp * hidden, ff, seed + 2)
    h = acts(n_tok * hidden, seed + 3).reshape(n_tok, hidden)
    if lg is None:
        lg = acts(n_tok * n_exp, seed + 4).reshape(n_tok, n_exp)
    out = torch.empty(n_tok, hidden, dtype=torch.float32, device="cuda")
    idx = torch.empty(n_tok, k, dtype=torch.int32, device="cuda")
    w = torch.empty(n_tok, k, dtype=torch.float32, device="cuda")
    engine.moe(tg, tg, td, dev(g), dev(u), dev(d), n_exp, k, hidden, ff, dev(lg), dev(h), n_tok, out, idx, w, ws=ws)
    torch.cuda.synchronize()
    want, widx, ww, mag = reference(tg, td, g, u, d, n_exp, k, hidden, ff, h, lg)
    assert np.array_equal(idx.cpu().numpy(), widx)
    np.testing.assert_allclose(w.cpu().numpy(), ww, rtol=2e-6, atol=1e-7)
    check_close(out.cpu().numpy(), want, mag)


@pytest.mark.parametrize("n_tok", [1, 3, 5, 8])
def test_moe_small(engine, n_tok):
    run(engine, le.Q4_K, le.Q6_K, 16, 4, 256, 256, n_tok, seed=10 + n_tok)


@pytest.mark.parametrize("tg,td", [(le.Q8_0, le.Q8_0), (le.IQ2_XXS, le.IQ3_XXS), (le.Q4_K, le.Q4_K)])
def test_moe_type_combos(engine, tg, td):
    run(engine, tg, td, 8, 2, 512, 256, 2, seed=40 + tg)


@pytest.mark.parametrize("tg,td", [(le.Q5_K, le.Q3_K), (le.Q4_0, le.Q4_0), (le.IQ2_S, le.Q5_K), (le.Q3_K, le.Q6_K),
                                   (le.Q4_K, le.Q5_K), (le.Q6_K, le.Q8_0)])
@pytest.mark.parametrize("n_tok", [1, 9, 70])
def test_moe_grouped_type_pairs(engine, tg, td, n_tok):
    """Type pairs without decode-shaped kernels (every pair of the nine types that the decode
    kernels do not take) run the grouped form at any token count."""
    print("moe type pair", tg, td, n_tok, flush=True)
    run(engine, tg, td, 16, 4, 512, 256, n_tok, seed=500 + tg + td + n_tok)


@pytest.mark.parametrize("n_tok", [1, 8])
def test_moe_config4(engine, n_tok):
    """Qwen3-30B-A3B shape: 128 experts, top-8, hidden 2048, ff 768, Q4_K gate/up, Q6_K down."""
    run(engine, le.Q4_K, le.Q6_K, 128, 8, 2048, 768, n_tok, seed=100 + n_tok)


@pytest.mark.parametrize("tg,td,n_tok,k", [(le.Q8_0, le.Q8_0, 2, 4), (le.Q8_0, le.Q8_0, 8, 4), (le.IQ2_XXS, le.IQ3_XXS, 8, 4)])
def test_moe_vector_down_images(engine, tg, td, n_tok, k):
    """The vector-ALU down kernel reads the pair images from LDS when they fit (2 tokens) and from
    the workspace when they do not (8 tokens x 4 experts at ff 768: 73 KB)."""
    run(engine, tg, td, 16, k, 512, 768, n_tok, seed=300 + n_tok + tg)


def test_moe_many_tokens_shared_experts(engine):
    """More tokens than fit one member pass (8), so expert groups loop over member chunks."""
    run(engine, le.Q4_K, le.Q6_K, 4, 2, 256, 256, 20, seed=77)


def test_moe_tied_logits_lower_index_first(engine):
    n_tok, n_exp, k = 2, 16, 4
    lg = np.zeros((n_tok, n_exp), dtype=np.float32)
    lg[0, [3, 9, 12]] = 1.5  # a three-way tie at the top
    lg[1, :] = 0.25          # every expert tied
    run(engine, le.Q4_K, le.Q6_K, n_exp, k, 256, 256, n_tok, seed=5, lg=lg)


def test_moe_tied_logits_staged(engine):
    """Ties on the single-launch path (hidden 2048, 128 experts, 4 tokens: one wave selects each
    token's top-k): equal logits go to the lower expert index, and -0 ties with +0."""
    n_tok, n_exp, k = 4, 128, 8
    lg = acts(n_tok * n_exp, 91).reshape(n_tok, n_exp).astype(np.float32)
    lg[0, [5, 64, 65, 127]] = 3.0            # tied at the top, across lanes and within a lane
    lg[1, :] = 0.5                           # every expert tied
    lg[2, :] = -1.0
    lg[2, [7, 100]] = 0.0
    lg[2, [3, 90]] = -0.0                    # -0 ties with +0: experts 3, 7, 90, 100 in index order
    lg[3, ::2] = 2.0                         # 64 tied, more than k
    run(engine, le.Q4_K, le.Q6_K, n_exp, k, 2048, 256, n_tok, seed=9, lg=lg)


def test_moe_errors(engine):
    import torch
    z = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    f = torch.zeros(4096, dtype=torch.float32, device="cuda")
    with pytest.raises(le.LeError) as e:
        engine.moe(le.Q4_K, le.Q8_0, le.Q6_K, z, z, z, 8, 2, 256, 256, f, f, 1, f)
    assert e.value.code == -2
    with pytest.raises(le.LeError) as e:
        engine.moe(le.Q4_K, le.Q4_K, le.Q6_K, z, z, z, 8, 2, 256, 256, f, f, 65537, f)
    assert e.value.code == -3
    with pytest.raises(le.LeError) as e:
        engine.moe(le.Q4_K, le.Q4_K, le.Q6_K, z, z, z, 8, 2, 256, 256, f, f, 1, f, ws=z, ws_bytes=16)
    assert e.value.code == -7


@pytest.mark.parametrize("hidden,ff,td,n_tok", [(1024, 256, le.Q6_K, 2), (3072, 512, le.Q6_K, 1), (2048, 768, le.Q4_K, 3),
                                                (2048, 256, le.Q6_K, 5), (1024, 768, le.Q4_K, 8)])
def test_moe_staged_shapes(engine, hidden, ff, td, n_tok):
    """The staged MFMA MoE kernels at each block shape they are built for (gate/up of 8 waves for
    hidden 2048, 4 waves for 1024 / 3072; down super-blocks per row 1..3)."""
    run(engine, le.Q4_K, td, 32, 4, hidden, ff, n_tok, seed=hidden + ff + n_tok)


def test_moe_staged_matches_vector_path(fresh_engine):
    """The staged MFMA kernels and the vector-ALU kernels agree on the same call."""
    import torch
    engine = fresh_engine
    n_exp, k, hidden, ff, n_tok = 64, 8, 2048, 768, 4
    g, _ = weights(le.Q4_K, n_exp * ff, hidden, 501)
    u, _ = weights(le.Q4_K, n_exp * ff, hidden, 502)
    d, _ = weights(le.Q6_K, n_exp * hidden, ff, 503)
    h = acts(n_tok * hidden, 504).reshape(n_tok, hidden)
    lg = acts(n_tok * n_exp, 505).reshape(n_tok, n_exp)
    outs = []
    for mfma in (1, 0):
        engine.set_option("moe_mfma", mfma)
        out = torch.empty(n_tok, hidden, dtype=torch.float32, device="cuda")
        engine.moe(le.Q4_K, le.Q4_K, le.Q6_K, dev(g), dev(u), dev(d), n_exp, k, hidden, ff, dev(lg), dev(h), n_tok, out)
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    engine.set_option("moe_mfma", 1)
    want, _, _, mag = reference(le.Q4_K, le.Q6_K, g, u, d, n_exp, k, hidden, ff, h, lg)
    check_close(outs[0], want, mag)
    check_close(outs[1], want, mag)


def test_moe_one_launch_repeated(engine):
    """The single-launch path (3+ tokens) reuses its device-wide barrier across calls: twenty calls
    in a row, every result checked against the oracle and bit-identical to the first."""
    import torch
    n_exp, k, hidden, ff, n_tok = 64, 8, 2048, 768, 6
    g, _ = weights(le.Q4_K, n_exp * ff, hidden, 601)
    u, _ = weights(le.Q4_K, n_exp * ff, hidden, 602)
    d, _ = weights(le.Q6_K, n_exp * hidden, ff, 603)
    h = acts(n_tok * hidden, 604).reshape(n_tok, hidden)
    lg = acts(n_tok * n_exp, 605).reshape(n_tok, n_exp)
    want, _, _, mag = reference(le.Q4_K, le.Q6_K, g, u, d, n_exp, k, hidden, ff, h, lg)
    dg, du, dd, dh, dl = dev(g), dev(u), dev(d), dev(h), dev(lg)
    out = torch.empty(n_tok, hidden, dtype=torch.float32, device="cuda")
    first = None
    for _ in range(20):
        out.fill_(float("nan"))
        engine.moe(le.Q4_K, le.Q4_K, le.Q6_K, dg, du, dd, n_exp, k, hidden, ff, dl, dh, n_tok, out)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        check_close(got, want, mag)
        # two blocks add into each output element of the down phase, onto zero: the same bits
        # in either order
        if first is None:
            first = got
        else:
            assert np.array_equal(got.view(np.uint32), first.view(np.uint32))


def test_moe_limits(engine):
    """The documented limits at their bounds: 64 tokens, top-16."""
    run(engine, le.Q4_K, le.Q6_K, 32, 16, 256, 256, 64, seed=700)


@pytest.mark.parametrize("n_tok", [10, 12, 16, 23, 64])
def test_moe_config4_more_tokens(engine, n_tok):
    """Config 4 beyond one call of the decode-shaped kernels: 8-token decode calls up to 10 tokens,
    the grouped form (each routed expert streamed once per tile of its pairs) from 11."""
    run(engine, le.Q4_K, le.Q6_K, 128, 8, 2048, 768, n_tok, seed=720 + n_tok)


@pytest.mark.parametrize("n_tok", [64, 256])
def test_moe_prefill_config4(engine, n_tok):
    """Config 4 on the grouped matrix-core form: route, group the pairs by expert, grouped gate /
    up / down matmuls, SwiGLU and the weighted combine."""
    run(engine, le.Q4_K, le.Q6_K, 128, 8, 2048, 768, n_tok, seed=800 + n_tok)


@pytest.mark.parametrize("tg,td", [(le.Q8_0, le.Q8_0), (le.IQ2_XXS, le.IQ3_XXS), (le.Q4_K, le.Q4_K), (le.Q6_K, le.Q6_K)])
def test_moe_prefill_types(engine, tg, td):
    run(engine, tg, td, 16, 4, 512, 512, 100, seed=820 + tg)


def test_moe_prefill_random_blocks(engine):
    """Arbitrary block bytes (bounded super-block scales) through the grouped form."""
    run(engine, le.Q4_K, le.Q6_K, 32, 4, 1024, 512, 130, seed=840, rand=True)


@pytest.mark.parametrize("tg,td", [(le.Q4_K, le.Q6_K), (le.IQ2_XXS, le.IQ3_XXS), (le.Q8_0, le.Q8_0)])
def test_moe_decode_random_blocks(engine, tg, td):
    """Arbitrary block bytes through the decode kernels (1 and 6 tokens)."""
    run(engine, tg, td, 32, 4, 1024, 512, 1, seed=860 + tg, rand=True)
    run(engine, tg, td, 32, 4, 1024, 512, 6, seed=870 + tg, rand=True)


def test_moe_prefill_uneven_experts(engine):
    """Most pairs on two experts, most experts empty; a token count that is not a tile multiple."""
    n_tok, n_exp, k = 300, 64, 2
    lg = acts(n_tok * n_exp, 880).reshape(n_tok, n_exp).astype(np.float32) * 0.01
    lg[:, 5] += 4.0
    lg[: n_tok // 2, 40] += 3.0
    lg[n_tok // 2:, 63] += 3.0
    run(engine, le.Q4_K, le.Q6_K, n_exp, k, 512, 256, n_tok, seed=881, lg=lg)


@pytest.mark.parametrize("n_tok", [17, 64])
def test_moe_prefill_matches_decode(fresh_engine, n_tok):
    """The grouped form and the decode kernels agree (both against the oracle) where both apply."""
    import torch
    engine = fresh_engine
    n_exp, k, hidden, ff = 64, 8, 2048, 768
    g, _ = weights(le.Q4_K, n_exp * ff, hidden, 901)
    u, _ = weights(le.Q4_K, n_exp * ff, hidden, 902)
    d, _ = weights(le.Q6_K, n_exp * hidden, ff, 903)
    h = acts(n_tok * hidden, 904).reshape(n_tok, hidden)
    lg = acts(n_tok * n_exp, 905).reshape(n_tok, n_exp)
    want, _, _, mag = reference(le.Q4_K, le.Q6_K, g, u, d, n_exp, k, hidden, ff, h, lg)
    for pre in (1, 0):
        engine.set_option("moe_prefill", pre)
        out = torch.empty(n_tok, hidden, dtype=torch.float32, device="cuda")
        engine.moe(le.Q4_K, le.Q4_K, le.Q6_K, dev(g), dev(u), dev(d), n_exp, k, hidden, ff, dev(lg), dev(h), n_tok, out)
        torch.cuda.synchronize()
        check_close(out.cpu().numpy(), want, mag)
    engine.set_option("moe_prefill", 1)


def test_moe_prefill_workspace(engine):
    """Above 64 tokens the call needs the prefill workspace; a decode-sized one is refused."""
    import torch
    n_exp, k, hidden, ff, n_tok = 16, 2, 256, 256, 80
    need = engine.moe_prefill_workspace_size(n_tok, k, n_exp, hidden, ff)
    assert need > engine.moe_workspace_size(n_tok, k, ff)
    z = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    f = torch.zeros(n_tok * max(hidden, n_exp), dtype=torch.float32, device="cuda")
    with pytest.raises(le.LeError) as e:
        engine.moe(le.Q4_K, le.Q4_K, le.Q6_K, z, z, z, n_exp, k, hidden, ff, f, f, n_tok, f, ws=z, ws_bytes=need - 1)
    assert e.value.code == -7


def test_moe_prefill_many_pairs(engine):
    """More than 16384 pairs (the grouping kernel's round): 2100 tokens at k = 8, and a hidden size
    that is not a multiple of the combine's 1024-column blocks."""
    run(engine, le.Q8_0, le.Q8_0, 16, 8, 1280, 256, 2100, seed=930)


@pytest.mark.parametrize("n_tok,k,n_exp", [(11, 8, 128), (20, 16, 256), (32, 16, 64), (32, 8, 200), (33, 8, 128), (12, 1, 3), (17, 2, 2)])
def test_moe_route_group_one_block(engine, n_tok, k, n_exp):
    """Routing and grouping in one block (up to 32 tokens and 1024 pairs) give the same bits as the
    per-token routing and per-expert grouping launches, including on tied logits."""
    import torch
    hidden, ff = 512, 256
    g = wbytes(le.Q4_K, n_exp * ff, hidden, 940)
    u = wbytes(le.Q4_K, n_exp * ff, hidden, 941)
    d = wbytes(le.Q6_K, n_exp * hidden, ff, 942)
    h = acts(n_tok * hidden, 943).reshape(n_tok, hidden)
    lg = np.round(acts(n_tok * n_exp, 944).reshape(n_tok, n_exp) * 4) / 4  # many ties
    ws = torch.empty(engine.moe_prefill_workspace_size(n_tok, k, n_exp, hidden, ff), dtype=torch.uint8, device="cuda")
    outs = []
    try:
        for r1 in (1, 0):
            engine.set_option("moe_route1", r1)
            out = torch.empty(n_tok, hidden, dtype=torch.float32, device="cuda")
            idx = torch.empty(n_tok, k, dtype=torch.int32, device="cuda")
            w = torch.empty(n_tok, k, dtype=torch.float32, device="cuda")
            engine.moe(le.Q4_K, le.Q4_K, le.Q6_K, dev(g), dev(u), dev(d), n_exp, k, hidden, ff, dev(lg), dev(h), n_tok,
                       out, idx, w, ws=ws)
            torch.cuda.synchronize()
            outs.append((out.cpu().numpy(), idx.cpu().numpy(), w.cpu().numpy()))
    finally:
        engine.set_option("moe_route1", 1)
    assert np.array_equal(outs[0][1], outs[1][1])
    assert np.array_equal(outs[0][2].view(np.uint32), outs[1][2].view(np.uint32))
    assert np.isfinite(outs[0][0]).all()
    assert np.array_equal(outs[0][0].view(np.uint32), outs[1][0].view(np.uint32))
    want, widx, _, mag = reference(le.Q4_K, le.Q6_K, g, u, d, n_exp, k, hidden, ff, h, lg)
    assert np.array_equal(outs[0][1], widx)
    check_close(outs[0][0], want, mag)


@pytest.mark.parametrize("n_tok", [1, 5])
def test_moe_grouped_form_few_tokens(engine, n_tok):
    """The grouped form forced down to 1 and 5 tokens (one-block routing and grouping with most
    waves holding no token) against the oracle."""
    import torch
    ws = torch.empty(engine.moe_prefill_workspace_size(n_tok, 8, 64, 512, 256), dtype=torch.uint8, device="cuda")
    try:
        engine.set_option("moe_prefill_min_tok", 1)
        run(engine, le.Q4_K, le.Q6_K, 64, 8, 512, 256, n_tok, seed=960 + n_tok, ws=ws)
    finally:
        engine.set_option("moe_prefill_min_tok", 11)
