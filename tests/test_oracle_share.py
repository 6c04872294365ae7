"""Pins of the oracle's top-k overlap (cross-layer top-k sharing statistics) against the reference's own torch
statement of it (sort, searchsorted, gather-compare: a different algorithm), python sets on tiny rows, and
invariants; and the host-side IndexShare pattern logic. CPU only."""
import os

import numpy as np
import pytest
import torch

from oracle import spmla_ref as ref


def _rows(L, n, K, R, seed, pad=0.1):
    g = np.random.default_rng(seed)
    base = g.permutation(R)[: 3 * K]
    s = np.stack([[g.choice(base, K, replace=False) for _ in range(n)] for _ in range(L)]).astype(np.int32)
    s[g.random(s.shape) < pad] = -1
    return s


def _torch_statement(sets):
    """index_share.py:113-118: sa = sort(a), pos = searchsorted(sa, sb) clamped, hit = sum((sa[pos] == sb) & sb >= 0)."""
    S = [torch.sort(torch.from_numpy(x).long(), dim=1).values for x in sets]
    L, n = len(S), S[0].shape[0]
    hits = np.zeros((L, L, n), dtype=np.int64)
    for a in range(L):
        for b in range(L):
            if a == b:
                continue
            sa, sb = S[a], S[b]
            pos = torch.searchsorted(sa, sb).clamp_(max=sa.shape[1] - 1)
            hits[a, b] = ((sa.gather(1, pos) == sb) & (sb >= 0)).sum(1).numpy()
    return hits


def test_overlap_vs_reference_statement():
    sets = _rows(4, 6, 300, 2000, seed=1)
    hits, nvalid = ref.topk_overlap(sets)
    assert np.array_equal(hits, _torch_statement(sets))
    assert np.array_equal(nvalid, (sets >= 0).sum(2))


def test_overlap_small_and_invariants():
    sets = np.array([[[1, 2, 3, -1], [5, 6, 7, 8]],
                     [[3, 2, 9, 10], [8, -1, -1, -1]],
                     [[1, 2, 3, -1], [11, 12, 13, 14]]], dtype=np.int32)
    hits, nvalid = ref.topk_overlap(sets)
    for i in range(2):
        for a in range(3):
            for b in range(3):
                if a != b:
                    A = {x for x in sets[a, i] if x >= 0}
                    assert hits[a, b, i] == sum(1 for x in sets[b, i] if x >= 0 and x in A)
    assert hits[0, 2, 0] == 3 == nvalid[0, 0]            # identical rows
    assert hits[0, 2, 1] == 0                           # disjoint rows
    assert hits[0, 1, 1] == 1 and hits[1, 0, 1] == 1
    big = _rows(3, 5, 200, 600, seed=2)
    h, nv = ref.topk_overlap(big)
    assert np.array_equal(h, h.transpose(1, 0, 2))
    assert np.all(h <= np.minimum(nv[:, None, :], nv[None, :, :]))


def test_index_share_pattern(tmp_path):
    from arcagi2_flashnext_dots3_amd.index_share import IndexShare
    dsa = [0, 1, 5, 9, 13]
    s = IndexShare("FSFSS", dsa)
    assert [s.skip(l) for l in dsa] == [False, True, False, True, True]
    assert [s.source_layer(l) for l in dsa] == [None, 0, None, 5, 5]
    with pytest.raises(ValueError):
        IndexShare("FSF", dsa).skip(0)                  # wrong length
    with pytest.raises(ValueError):
        IndexShare("FXFFF", dsa).skip(0)
    assert not IndexShare("SSSSS", dsa).skip(0)          # the first DSA layer always runs its indexer
    f = tmp_path / "pat.txt"
    f.write_text("FFFFF")
    s = IndexShare("@" + str(f), dsa)
    assert not s.skip(5)
    f.write_text("FFSFF")
    os.utime(f, ns=(1, 10 ** 19))                        # a new mtime: the file is read again
    assert s.skip(5)
    os.remove(f)
    assert not s.skip(5)                                 # file gone: nothing skipped


def test_share_wrapper_skips_and_reuses():
    from arcagi2_flashnext_dots3_amd.index_share import IndexShare, wrap
    calls = []
    buf = torch.zeros(2, 4, dtype=torch.int32)

    def indexer(lid, x):
        calls.append(lid)
        buf.fill_(lid)
        return buf

    fwd = wrap(indexer, share=IndexShare("FSF", [0, 3, 7]), topk_buffer=lambda: buf)
    assert int(fwd(0, None)[0, 0]) == 0
    assert int(fwd(3, None)[0, 0]) == 0                  # skipped: layer 0's top-k left in place
    assert int(fwd(7, None)[0, 0]) == 7
    assert calls == [0, 7]
