"""The no-allocation top-k entry point (spmla_topk_scratch, the library's fixed per-GPU scratch in place of a caller
workspace) against the workspace entry point it varies (spmla_topk_ws) through the C-ABI: bit-exact indices on two
calls in a row, the second smaller, so that the second runs over the first call's leftover scratch contents; the
oracle checks the first call's result too."""
import numpy as np
import pytest
import torch

from oracle import spmla_ref as ref

pytestmark = pytest.mark.gpu


def _logits(rows, L, seed):
    g = torch.Generator().manual_seed(seed)
    lg = torch.randn(rows, L, generator=g)
    lg[:, ::7] = lg[:, 3:4]                       # ties across each row (lower column must win)
    ctx = torch.randint(L // 2, L + 1, (rows,), generator=g).to(torch.int32)
    ctx[0] = L
    return lg.contiguous(), ctx


def test_topk_scratch_matches_workspace(dev):
    from arcagi2_flashnext_dots3_amd import _lib, kernels
    lib = _lib.lib()
    assert lib.spmla_topk_scratch_bytes() == 16 << 20
    for step, (rows, L, K) in enumerate([(64, 131072, 2048), (9, 20000, 1024)]):
        lg, ctx = _logits(rows, L, 40 + step)
        print(f"[no-alloc topk] call {step}: rows={rows} L={L} K={K}", flush=True)
        # (the first call's overflow lists do not fit the scratch: it runs without them, re-reading the row at the
        # second level, while the workspace path below uses them; both are exact)
        dl, dc = lg.to(dev), ctx.to(dev)
        got = kernels.topk_scratch(dl, dc, K)
        exp = kernels.topk(dl, dc, K)                 # spmla_topk_ws with its own workspace
        torch.cuda.synchronize()
        g, e = got.cpu().numpy(), exp.cpu().numpy()
        assert np.array_equal(g, e), f"call {step}: scratch path differs from the workspace path"
        if step == 0:                                 # and the workspace path against the oracle on a few rows
            sub = [0, 1, 63]
            o = ref.topk(lg.numpy()[sub], ctx.numpy()[sub], K)
            assert np.array_equal(g[sub], o)


def test_topk_scratch_rejects_oversize(dev):
    from arcagi2_flashnext_dots3_amd import _lib, kernels
    lib = _lib.lib()
    rows, L, K = 256, 131072, 2048                  # 256 x 112 KiB of workspace > 16 MiB, even without overflow lists
    assert lib.spmla_topk_ws_bytes(rows, L, K) > lib.spmla_topk_scratch_bytes()
    lg = torch.zeros(rows, L, device=dev)
    ctx = torch.full((rows,), L, dtype=torch.int32, device=dev)
    with pytest.raises(RuntimeError, match="-5"):
        kernels.topk_scratch(lg, ctx, K)
