"""Pins of the oracle's MTP request union (python sets on tiny requests; the order by its definition). CPU only."""
import numpy as np

from oracle import spmla_ref as ref


def test_union_tiny_by_hand():
    idx = np.array([[5, 7, 9, -1], [7, 3, 5, 11], [9, 9 + 100, 5, 2],      # request 0: 3 tokens (row 109 >= R)
                    [1, 2, 3, 4], [4, 3, 2, 1]], dtype=np.int32)            # request 1: 2 tokens, same rows
    u, mk, cnt = ref.mtp_union(idx, T=5, ql=3, cu=None, nreq=2, R=100, nmax=12)
    # request 0: 5 -> tokens 0,1,2 (7); 7 -> 0,1 (3); 9 -> 0,2 (5); 3 -> 1 (2); 11 -> 1 (2); 2 -> 2 (4)
    assert cnt.tolist() == [6, 4]
    assert u[0, :6].tolist() == [5, 9, 2, 7, 3, 11] and mk[0, :6].tolist() == [7, 5, 4, 3, 2, 2]
    assert np.all(u[0, 6:] == -1)
    assert u[1, :4].tolist() == [1, 2, 3, 4] and mk[1, :4].tolist() == [3, 3, 3, 3]


def test_union_random_sets():
    g = np.random.default_rng(0)
    T, topk, R = 10, 64, 300
    idx = np.stack([g.choice(R + 20, topk, replace=False) for _ in range(T)]).astype(np.int32) - 10
    cu = np.array([0, 4, 4, 7, 10])
    u, mk, cnt = ref.mtp_union(idx, T, None, cu, 4, R, nmax=6 * topk)
    for r in range(4):
        rows = idx[cu[r]:cu[r + 1]]
        sel = {int(h) for h in rows.reshape(-1) if 0 <= h < R}
        got = u[r, :cnt[r]].tolist()
        assert len(got) == len(set(got)) and set(got) == sel
        for h, m in zip(got, mk[r, :cnt[r]]):
            assert m == sum(1 << j for j in range(rows.shape[0]) if h in set(rows[j].tolist()))
        keys = [(-int(m), min(j * topk + int(np.nonzero(rows[j] == h)[0][0]) for j in range(rows.shape[0])
                              if h in set(rows[j].tolist()))) for h, m in zip(got, mk[r, :cnt[r]])]
        assert keys == sorted(keys)
    assert cnt[1] == 0 and np.all(u[1] == -1)
