"""le_gemm_noalloc (workspace from the library's per-GPU scratch array) against le_gemm (caller
workspace): same kernels, so with one K slice the outputs are bit-identical; both are also checked
against the oracle's matmat. Two calls in a row, the second smaller, show that the shared scratch
carries nothing over from the previous call."""
import numpy as np
import pytest

import lastengine_amd as le
import oracle
from tests.util import weights, acts, check_close

pytestmark = pytest.mark.gpu


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _pair(eng, ty, rows, cols, m, seed):
    import torch
    q, _ = weights(ty, rows, cols, seed=seed)
    x = acts(m * cols, seed + 1)
    dq, dx = dev(q), dev(x)
    y_ws = torch.full((m * rows,), float("nan"), dtype=torch.float32, device="cuda")
    y_na = torch.full((m * rows,), float("nan"), dtype=torch.float32, device="cuda")
    eng.gemm(ty, dq, dx, m, y_ws, rows, cols)
    eng.gemm_noalloc(ty, dq, dx, m, y_na, rows, cols)
    torch.cuda.synchronize()
    return q, x, y_ws.cpu().numpy(), y_na.cpu().numpy()


@pytest.mark.parametrize("name", ["Q4_K"])
def test_noalloc_matches_gemm_two_calls(fresh_engine, name):
    ty = le.TYPES[name]
    fresh_engine.set_option("gm_ksplit", 1)  # one K slice: no atomics, reproducible bits
    fresh_engine.set_option("gq_ksplit", 1)
    for (rows, cols, m, seed) in [(2048, 4096, 64, 11), (1024, 2048, 20, 12)]:
        print("noalloc case", name, rows, cols, m, flush=True)
        q, x, y_ws, y_na = _pair(fresh_engine, ty, rows, cols, m, seed)
        assert np.array_equal(y_ws.view(np.uint32), y_na.view(np.uint32)), "noalloc differs from le_gemm"
        want = oracle.matmat(ty, q, rows, cols, x.reshape(m, cols))
        w = oracle.dequant_rows(ty, q, rows, cols).astype(np.float64)
        mag = np.abs(x.reshape(m, cols).astype(np.float64)) @ np.abs(w).T
        check_close(y_na.reshape(m, rows), want, mag)


def test_noalloc_default_options_and_few_tokens(engine):
    """Default launch policy (K split where chosen: the scratch holds the slices' partial results,
    as does the workspace le_gemm gets here, so both sum them in the same order and agree bit for
    bit) and a token count that needs no workspace: both agree with the oracle."""
    ty = le.Q4_K
    for (rows, cols, m, seed) in [(1024, 4096, 48, 21), (512, 4096, 8, 22)]:
        print("noalloc default case", rows, cols, m, flush=True)
        q, x, y_ws, y_na = _pair(engine, ty, rows, cols, m, seed)
        if m > 16:
            assert np.array_equal(y_ws.view(np.uint32), y_na.view(np.uint32)), "noalloc differs from le_gemm"
        want = oracle.matmat(ty, q, rows, cols, x.reshape(m, cols))
        w = oracle.dequant_rows(ty, q, rows, cols).astype(np.float64)
        mag = np.abs(x.reshape(m, cols).astype(np.float64)) @ np.abs(w).T
        check_close(y_na.reshape(m, rows), want, mag)
        check_close(y_ws.reshape(m, rows), want, mag)


def test_noalloc_rejects_sizes_above_scratch(engine):
    import torch
    m, cols, rows = 2048, 8192, 256  # 64 MiB of activation planes > 32 MiB of scratch
    assert engine.gemm_workspace_size(le.Q4_K, m, cols) > 32 << 20
    w = torch.zeros(rows * le.row_bytes(le.Q4_K, cols), dtype=torch.uint8, device="cuda")
    x = torch.zeros(m * cols, dtype=torch.float32, device="cuda")
    y = torch.zeros(m * rows, dtype=torch.float32, device="cuda")
    with pytest.raises(le.LeError) as ei:
        engine.gemm_noalloc(le.Q4_K, w, x, m, y, rows, cols)
    assert ei.value.code == -7
    assert "scratch" in str(ei.value)
