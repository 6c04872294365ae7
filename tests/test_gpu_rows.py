"""GPU parity of the row plumbing: top-k -> global rows, gather (bytes), row copy, tier split, compact stage."""
import numpy as np
import pytest
import torch

from oracle import spmla_ref as ref

pytestmark = pytest.mark.gpu


def test_rows_from_topk(dev):
    from arcagi2_flashnext_dots3_amd import kernels
    g = np.random.default_rng(0)
    T, K, bs, cols, nb = 20, 300, 64, 40, 900
    bt = g.integers(-1, nb, (8, cols)).astype(np.int32)
    req = g.integers(0, 8, T).astype(np.int32)
    tk = g.integers(-1, cols * bs + 50, (T, K)).astype(np.int32)
    counts = torch.zeros(T, dtype=torch.int32, device=dev)
    rows = kernels.rows_from_topk(torch.from_numpy(tk).to(dev), torch.from_numpy(req).to(dev),
                                  torch.from_numpy(bt).to(dev), bs, counts=counts)
    exp = ref.rows_from_topk(tk, req, bt, bs)
    assert np.array_equal(rows.cpu().numpy(), exp)
    assert np.array_equal(counts.cpu().numpy(), (exp >= 0).sum(1))


def test_gather_and_copy(dev):
    from arcagi2_flashnext_dots3_amd import kernels
    g = np.random.default_rng(1)
    R, n = 5000, 3000
    src = g.integers(0, 256, (R, 656)).astype(np.uint8)
    rows = g.integers(-3, R + 3, n).astype(np.int64)
    out = torch.full((n, 656), 7, dtype=torch.uint8, device=dev)
    kernels.gather(torch.from_numpy(src).to(dev), torch.from_numpy(rows).to(dev), out)
    assert np.array_equal(out.cpu().numpy(), ref.gather(src, rows))
    dst = torch.zeros(800, 656, dtype=torch.uint8, device=dev)
    sr = g.permutation(R)[:800].astype(np.int64)
    dr = g.permutation(800).astype(np.int64)
    kernels.copy_rows(torch.from_numpy(src).to(dev), torch.from_numpy(sr).to(dev), dst, torch.from_numpy(dr).to(dev))
    exp = np.zeros((800, 656), dtype=np.uint8)
    exp[dr] = src[sr]
    assert np.array_equal(dst.cpu().numpy(), exp)


def test_gather_from_pinned_host(dev):
    from arcagi2_flashnext_dots3_amd import kernels
    g = np.random.default_rng(2)
    R, n = 4096, 1000
    host = torch.from_numpy(g.integers(0, 256, (R, 656)).astype(np.uint8)).pin_memory()
    rows = torch.from_numpy(g.integers(0, R, n).astype(np.int64))
    out = torch.empty(n, 656, dtype=torch.uint8, device=dev)
    kernels.gather(host, rows.to(dev), out)           # kernel reads pinned host memory over PCIe
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), host.numpy()[rows.numpy()])


@pytest.mark.parametrize("T,K,zero0", [(9, 300, False), (1100, 7, True)])
def test_gather_tiers(dev, T, K, zero0):
    """Host-tier staging from pinned memory: rows k < counts[t] of each token land at t * K + k, out-of-range rows as
    zero rows, untouched rows keep their bytes, row 0 is zeroed when token 0 has none (T > 1024: two token chunks)."""
    from arcagi2_flashnext_dots3_amd import kernels
    g = np.random.default_rng(7)
    R = 3000
    host = torch.from_numpy(g.integers(0, 256, (R, 656)).astype(np.uint8)).pin_memory()
    rows = g.integers(-2, R + 2, (T, K)).astype(np.int32)
    counts = g.integers(-1, K + 3, T).astype(np.int32)
    counts[0] = 0 if zero0 else K
    out = torch.full((T * K, 656), 9, dtype=torch.uint8, device=dev)
    kernels.gather_tiers(host, torch.from_numpy(rows).to(dev), torch.from_numpy(counts).to(dev), out)
    torch.cuda.synchronize()
    exp = np.full((T * K, 656), 9, dtype=np.uint8)
    for t in range(T):
        for k in range(min(max(int(counts[t]), 0), K)):
            r = int(rows[t, k])
            exp[t * K + k] = host.numpy()[r] if 0 <= r < R else 0
    if zero0:
        exp[0] = 0
    assert np.array_equal(out.cpu().numpy(), exp)


@pytest.mark.parametrize("K", [2048, 300, 5000])
def test_tier_split(dev, K):
    """One and several 2048-entry chunks per token, a K that is not a multiple of 8; rowmap entries with negative
    values other than -1 count as host rows."""
    from arcagi2_flashnext_dots3_amd import kernels
    g = np.random.default_rng(3)
    T, R = 9, 50000
    rowmap = np.full(R, -1, dtype=np.int32)
    hot = g.permutation(R)[: R // 4]
    rowmap[hot] = np.arange(hot.size, dtype=np.int32)
    rowmap[g.permutation(R)[:100]] = -7
    idx = g.integers(-2, R + 2, (T, K)).astype(np.int32)
    out = kernels.tier_split(torch.from_numpy(idx).to(dev), torch.from_numpy(rowmap).to(dev), R)
    exp = ref.tier_split(idx, rowmap, R)
    for a, b in zip(out, exp):
        assert np.array_equal(a.cpu().numpy(), b)


def test_compact_stage(dev):
    from arcagi2_flashnext_dots3_amd import kernels
    g = np.random.default_rng(4)
    tot, M, K = 70000, 64, 2048
    rows = g.integers(0, 10 ** 7, tot).astype(np.int64)
    sidx = g.integers(-1, tot, (M, K)).astype(np.int32)
    sel, U, sidx2 = kernels.compact_stage(torch.from_numpy(rows).to(dev), torch.from_numpy(sidx).to(dev))
    es, e2 = ref.compact_stage(rows, sidx)
    u = int(U.item())
    assert u == es.size
    assert np.array_equal(sel.cpu().numpy()[:u], es)
    assert np.array_equal(sidx2.cpu().numpy(), e2)
