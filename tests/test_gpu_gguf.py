"""Tensors read from a GGUF file (include/le_gguf.h) feed the device kernels: the 3D
ffn_{gate,up,down}_exps tensors of a Qwen3-MoE-shaped layer (as cpu_ref::Model reads them,
src/cpu_ref.rs:70-85) go to le_moe_layer as whole slabs and through a pointer table of per-expert
slabs (the reference's expert arena, src/gpu.rs:587-596), and a 2D tensor goes to le_matvec; each
against the oracle on the same bytes."""
import numpy as np
import pytest

import lastengine_amd as le
import oracle
from lastengine_amd.gguf import Gguf
from tests import gguf_writer as W
from tests.test_gpu_moe import reference
from tests.util import acts, check_close, weights

pytestmark = pytest.mark.gpu


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    n_exp, hidden, ff = 32, 2048, 768
    g, _ = weights(le.Q4_K, n_exp * ff, hidden, 501)
    u, _ = weights(le.Q4_K, n_exp * ff, hidden, 502)
    d, _ = weights(le.Q6_K, n_exp * hidden, ff, 503)
    o, _ = weights(le.Q8_0, 1000, hidden, 504)
    path = str(tmp_path_factory.mktemp("m") / "moe.gguf")
    W.write(path, [("general.architecture", W.STR, "qwen3moe"), ("qwen3moe.expert_count", W.U32, n_exp),
                   ("qwen3moe.expert_used_count", W.U32, 8), ("qwen3moe.embedding_length", W.U32, hidden),
                   ("qwen3moe.expert_feed_forward_length", W.U32, ff)],
            [("blk.0.ffn_gate_exps.weight", [hidden, ff, n_exp], le.Q4_K, g),
             ("blk.0.ffn_up_exps.weight", [hidden, ff, n_exp], le.Q4_K, u),
             ("blk.0.ffn_down_exps.weight", [ff, hidden, n_exp], le.Q6_K, d),
             ("output.weight", [hidden, 1000], le.Q8_0, o)])
    return path


@pytest.mark.parametrize("n_tok", [1, 8])
@pytest.mark.parametrize("via_ptrs", [False, True])
def test_moe_from_gguf(engine, model, n_tok, via_ptrs):
    import torch
    gf = Gguf(model)
    n_exp, k, hidden, ff = (gf.as_u64("qwen3moe.expert_count"), gf.as_u64("qwen3moe.expert_used_count"),
                            gf.as_u64("qwen3moe.embedding_length"), gf.as_u64("qwen3moe.expert_feed_forward_length"))
    names = ["blk.0.ffn_%s_exps.weight" % p for p in ("gate", "up", "down")]
    host = [gf.tensor_bytes(n) for n in names]
    tys = [gf.find(n).ggml_type for n in names]
    h = acts(n_tok * hidden, 77 + n_tok).reshape(n_tok, hidden)
    lg = acts(n_tok * n_exp, 88 + n_tok).reshape(n_tok, n_exp)
    out = torch.empty(n_tok, hidden, dtype=torch.float32, device="cuda")
    idx = torch.empty(n_tok, k, dtype=torch.int32, device="cuda")
    w = torch.empty(n_tok, k, dtype=torch.float32, device="cuda")
    if via_ptrs:
        # every expert's slab as its own device buffer, addressed through pointer tables
        slabs = [[dev(gf.read(*gf.expert_slab(n, e))) for e in range(n_exp)] for n in names]
        tabs = [dev(np.array([s.data_ptr() for s in ss], dtype=np.uint64)) for ss in slabs]
        engine.moe_ptrs(tys[0], tys[1], tys[2], tabs[0], tabs[1], tabs[2], n_exp, k, hidden, ff, dev(lg), dev(h), n_tok,
                        out, idx, w)
    else:
        engine.moe(tys[0], tys[1], tys[2], dev(host[0]), dev(host[1]), dev(host[2]), n_exp, k, hidden, ff, dev(lg), dev(h),
                   n_tok, out, idx, w)
    torch.cuda.synchronize()
    want, widx, ww, mag = reference(tys[0], tys[2], host[0], host[1], host[2], n_exp, k, hidden, ff, h, lg)
    assert np.array_equal(idx.cpu().numpy(), widx)
    np.testing.assert_allclose(w.cpu().numpy(), ww, rtol=2e-6, atol=1e-7)
    check_close(out.cpu().numpy(), want, mag)


def test_matvec_from_gguf(engine, model):
    import torch
    gf = Gguf(model)
    t = gf.find("output.weight")
    cols, rows = t.dims
    q = gf.tensor_bytes("output.weight")
    x = acts(cols, 99)
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    engine.mv(t.ggml_type, dev(q), dev(x), y, rows, cols)
    torch.cuda.synchronize()
    want = oracle.matvec(t.ggml_type, q, rows, cols, x)
    wd = oracle.dequant_rows(t.ggml_type, q, rows, cols).astype(np.float64)
    check_close(y.cpu().numpy(), want, np.abs(wd) @ np.abs(x.astype(np.float64)))
