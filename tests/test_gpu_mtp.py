"""GPU parity of the MTP request union (spmla_mtp_union) vs the oracle, bit-exact (rows, masks, counts, order)."""
import numpy as np
import pytest
import torch

from oracle import spmla_ref as ref
from tests.helpers import attn_excess

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("ql,T,topk,R,shared", [(4, 64, 2048, 1 << 20, 0.8), (3, 10, 512, 5000, 0.5),
                                                 (6, 12, 2048, 4096, 0.3), (1, 5, 100, 1000, 0.0)])
def test_mtp_union(dev, ql, T, topk, R, shared):
    from arcagi2_flashnext_dots3_amd import kernels
    g = np.random.default_rng(topk + ql)
    idx = np.empty((T, topk), dtype=np.int32)
    for r0 in range(0, T, ql):
        base = g.choice(R, topk, replace=False)
        for t in range(r0, min(r0 + ql, T)):
            own = g.choice(R, topk, replace=False)
            row = np.where(g.random(topk) < shared, base, own)
            _, first = np.unique(row, return_index=True)
            keep = np.zeros(topk, bool)
            keep[first] = True
            idx[t] = np.where(keep, row, -1)                          # distinct within a token
    idx[g.random(idx.shape) < 0.02] = R + 7                            # invalid rows
    print(f"[mtp union] ql={ql} T={T} topk={topk}", flush=True)
    u, mk, cnt = kernels.mtp_union(torch.from_numpy(idx).to(dev), ql=ql, R=R)
    torch.cuda.synchronize()
    nreq = (T + ql - 1) // ql
    eu, emk, ecnt = ref.mtp_union(idx, T, ql, None, nreq, R, nmax=u.shape[1], gmax=min(ql, 6))
    assert np.array_equal(cnt.cpu().numpy(), ecnt)
    assert np.array_equal(u.cpu().numpy(), eu)
    got_mk = mk.cpu().numpy()
    for r in range(nreq):
        assert np.array_equal(got_mk[r, :ecnt[r]], emk[r, :ecnt[r]])


def test_mtp_union_boundaries(dev):
    from arcagi2_flashnext_dots3_amd import kernels
    g = np.random.default_rng(9)
    T, topk, R = 9, 256, 2000
    idx = np.stack([g.choice(R, topk, replace=False) for _ in range(T)]).astype(np.int32)
    cu = np.array([0, 2, 2, 8], dtype=np.int32)                        # an empty request; one of 6 tokens
    u, mk, cnt = kernels.mtp_union(torch.from_numpy(idx).to(dev), cu=torch.from_numpy(cu).to(dev), R=R,
                                   max_query_len=6)
    torch.cuda.synchronize()
    eu, emk, ecnt = ref.mtp_union(idx, T, None, cu, 3, R, nmax=u.shape[1])
    assert np.array_equal(cnt.cpu().numpy(), ecnt) and np.array_equal(u.cpu().numpy(), eu)
    # a host-declared request of 7 tokens is refused (the kernels take at most 6), as is cu without its maximum
    with pytest.raises(ValueError, match="at most 6"):
        kernels.mtp_union(torch.from_numpy(idx).to(dev), cu=torch.tensor([0, 2, 9], dtype=torch.int32, device=dev),
                          R=R, max_query_len=7)
    with pytest.raises(ValueError, match="max_query_len"):
        kernels.mtp_union(torch.from_numpy(idx).to(dev), cu=torch.from_numpy(cu).to(dev), R=R)


def _mtp_inputs(B, ql, H, R, K, shared, seed):
    from tests.helpers import make_pool_656, make_q
    g = np.random.default_rng(seed)
    T = B * ql
    idx = np.empty((T, K), dtype=np.int32)
    for b in range(B):
        base = g.choice(R, K, replace=False)
        for t in range(b * ql, (b + 1) * ql):
            own = g.choice(R, K, replace=False)
            row = np.where(g.random(K) < shared, base, own)
            _, first = np.unique(row, return_index=True)
            keep = np.zeros(K, bool)
            keep[first] = True
            idx[t] = np.where(keep, row, -1)
    pool, _, _ = make_pool_656(R, seed=seed + 1)
    return torch.from_numpy(idx), pool, make_q(T, H, seed=seed + 2)


@pytest.mark.parametrize("B,ql,H,K,shared,split", [(4, 4, 128, 1024, 0.8, 1), (3, 3, 64, 512, 0.5, 1),
                                                   (2, 2, 128, 2048, 0.9, 2), (5, 1, 32, 256, 0.0, 1)])
def test_attend_packed_vs_oracle_and_per_token(dev, B, ql, H, K, shared, split):
    from arcagi2_flashnext_dots3_amd import kernels
    R = 8192
    idx, pool, q = _mtp_inputs(B, ql, H, R, K, shared, seed=K + ql)
    idx[0, :7] = R + 3                                                  # invalid rows
    sm = 192 ** -0.5
    print(f"[packed] B={B} ql={ql} H={H} K={K} split={split}", flush=True)
    pd = torch.from_numpy(pool).to(dev)
    out, lse = kernels.attend_packed(q.to(dev), pd, idx.to(dev), sm, ql=ql, split=split)
    o1, l1 = kernels.attend(q.to(dev), pd, idx.to(dev), sm)
    torch.cuda.synchronize()
    o_ref, l_ref = ref.attention(q.float().numpy(), pool, idx.numpy(), sm)
    o = out.float().cpu().numpy()
    l = lse.cpu().numpy()
    err_o = attn_excess(o, o_ref)
    err_l = np.abs(l - l_ref).max()
    print(f"[packed] vs oracle: excess over the output bar {err_o:.3e}, lse {err_l:.3e}", flush=True)
    assert err_o <= 0 and err_l <= 1e-3
    d = ((out.float() - o1.float()).abs() / o1.float().abs().clamp_min(1.0)).max()
    assert float(d) <= 1e-2 and float((lse - l1).abs().max()) <= 1e-4


def test_attend_packed_variable_requests(dev):
    """cu boundaries: requests of 3, 1, 0 and 6 tokens, every token computed; a request of 7 tokens is refused."""
    from arcagi2_flashnext_dots3_amd import kernels
    H, R, K = 64, 4096, 512
    idx, pool, q = _mtp_inputs(1, 10, H, R, K, 0.7, seed=5)
    cu = torch.tensor([0, 3, 4, 4, 10], dtype=torch.int32)
    sm = 192 ** -0.5
    pd = torch.from_numpy(pool).to(dev)
    out = torch.full((10, H, 512), 7.0, dtype=torch.bfloat16, device=dev)
    lse = torch.full((10, H), 7.0, dtype=torch.float32, device=dev)
    kernels.attend_packed(q.to(dev), pd, idx.to(dev), sm, cu=cu.to(dev), out=out, lse=lse, max_query_len=6)
    torch.cuda.synchronize()
    o_ref, l_ref = ref.attention(q.float().numpy(), pool, idx.numpy(), sm)
    o = out.float().cpu().numpy()
    l = lse.cpu().numpy()
    assert attn_excess(o, o_ref) <= 0
    assert np.abs(l - l_ref).max() <= 1e-3
    with pytest.raises(ValueError, match="at most 6"):
        kernels.attend_packed(q.to(dev), pd, idx.to(dev), sm, cu=torch.tensor([0, 3, 10], dtype=torch.int32,
                                                                               device=dev), max_query_len=7)
