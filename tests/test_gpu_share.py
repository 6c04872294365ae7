"""GPU parity of spmla_topk_overlap (cross-layer top-k overlap counts) against the oracle, bit-exact (integer
counts), and the TopkOverlap accumulation built on it against the same statistic computed from the oracle."""
import numpy as np
import pytest
import torch

from oracle import spmla_ref as ref

pytestmark = pytest.mark.gpu


def _sets(L, n, K, R, seed):
    g = np.random.default_rng(seed)
    base = g.permutation(R)[: 2 * K]                       # shared pool: substantial overlaps
    s = np.stack([[g.choice(base, K, replace=False) for _ in range(n)] for _ in range(L)]).astype(np.int32)
    s[g.random(s.shape) < 0.05] = -1
    s[0, 0] = -1                                            # an empty row
    if n > 1:
        s[1, 1] = s[0, 1]                                   # identical rows
    return s


@pytest.mark.parametrize("L,n,K", [(5, 40, 2048), (13, 8, 512), (2, 3, 7)])
def test_topk_overlap(dev, L, n, K):
    from arcagi2_flashnext_dots3_amd import kernels
    sets = _sets(L, n, K, 100000, seed=L + n)
    print(f"[overlap] L={L} n={n} K={K}", flush=True)
    hits, nvalid = kernels.topk_overlap(torch.from_numpy(sets).to(dev))
    torch.cuda.synchronize()
    eh, ev = ref.topk_overlap(sets)
    assert np.array_equal(hits.cpu().numpy(), eh) and np.array_equal(nvalid.cpu().numpy(), ev)


def test_overlap_recorder(dev, tmp_path):
    from arcagi2_flashnext_dots3_amd.index_share import BINS, TopkOverlap
    dsa = [0, 1, 5]
    L, n, K = 3, 20, 256
    sets = _sets(L, n, K, 5000, seed=3)
    ctx = np.random.default_rng(4).integers(100, 40000, n)
    rec = TopkOverlap(str(tmp_path), dsa)
    for l, lid in enumerate(dsa):
        rec.record(lid, torch.from_numpy(sets[l]).to(dev), torch.from_numpy(ctx).to(dev))
    z = np.load(tmp_path / "overlap_rank0.npz")
    eh, ev = ref.topk_overlap(sets)
    nv = np.maximum(ev, 1).astype(np.float64)
    b = np.searchsorted(np.array(BINS[1:-1]), ctx, side="left")
    want = np.zeros((len(BINS) - 1, L, L))
    for i in range(n):
        for a in range(L):
            for c in range(L):
                if a != c:
                    want[b[i], a, c] += eh[a, c, i] / nv[c, i]
    assert np.allclose(z["sum_rec"], want, rtol=1e-12, atol=1e-12)
    assert np.array_equal(z["cnt"], np.bincount(b, minlength=len(BINS) - 1).astype(np.float64))
