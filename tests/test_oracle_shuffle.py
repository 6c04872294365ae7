"""Pins of the oracle's SHUFFLE indexer-cache layout (the reference reader's byte offsets written out element by
element), its round trip, the key write into it, and the paged reader's per-row context rule. CPU only."""
import numpy as np
import torch

from oracle import spmla_ref as ref
from tests.helpers import bf16_bits


def test_shuffle_layout_positions():
    bs, nb = 32, 2
    g = np.random.default_rng(0)
    rows = g.integers(0, 256, (nb * bs, 132)).astype(np.uint8)
    cache = ref.shuffle_layout(rows, bs)
    assert cache.shape == (nb, bs * 132)
    for b in range(nb):
        for t in range(bs):
            for d in range(128):
                # dsa_sm89.py:65 koff = (t // 16) * (16 * D) + (t % 16) * 16 + (d // 16) * 256 + d % 16, D = 128
                assert cache[b, (t // 16) * 16 * 128 + (t % 16) * 16 + (d // 16) * 256 + d % 16] == rows[b * bs + t, d]
            # dsa_sm89.py:67: scale = kv32[(BS * D) // 4 + t] (fp32 view of the block)
            assert np.array_equal(cache[b, bs * 128 + 4 * t: bs * 128 + 4 * t + 4], rows[b * bs + t, 128:132])
    assert np.array_equal(ref.shuffle_rows(cache, bs), rows)


def test_key_write_shuffle_equals_row_write():
    bs, nb = 16, 3
    k = bf16_bits(torch.randn(40, 128, generator=torch.Generator().manual_seed(1)) * 3)
    slots = np.array(list(range(0, 80, 2)))
    slots[5] = -1
    slots[7] = nb * bs + 4                              # beyond the cache: skipped
    rows = np.zeros((nb * bs, 132), dtype=np.uint8)
    ref.index_key_write(k, slots, rows)
    cache = np.zeros((nb, bs * 132), dtype=np.uint8)
    ref.index_key_write_shuffle(k, slots, cache, bs)
    assert np.array_equal(cache, ref.shuffle_layout(rows, bs))


def test_paged_ctx_rule():
    req, ctx = ref.paged_ctx(np.array([10, 20]), 3)
    assert req.tolist() == [0, 0, 0, 1, 1, 1] and ctx.tolist() == [8, 9, 10, 18, 19, 20]
    req, ctx = ref.paged_ctx(np.array([[5, 6], [7, 8]]), 2)
    assert req.tolist() == [0, 0, 1, 1] and ctx.tolist() == [5, 6, 7, 8]


def test_paged_logits_unclamped_and_matches_row_store():
    bs, nb, B, nn, L = 16, 6, 2, 2, 64
    g = torch.Generator().manual_seed(2)
    k = bf16_bits(torch.randn(nb * bs, 128, generator=g) * 50)
    rows = np.zeros((nb * bs, 132), dtype=np.uint8)
    ref.index_key_write(k, np.arange(nb * bs), rows)
    cache = ref.shuffle_layout(rows, bs)
    q = torch.randn(B, nn, 64, 128, generator=g).float().numpy() * 40
    w = torch.rand(B * nn, 64, generator=g).numpy()
    bt = np.array([[5, 2, 0, 1], [3, 4, 1, 0]], dtype=np.int32)
    sl = np.array([50, 64])
    got = ref.paged_mqa_logits(q, cache, w, sl, bt, bs, L)
    req, ctx = ref.paged_ctx(sl, nn)
    want = ref.index_logits(q.reshape(B * nn, 64, 128), w, rows, bt, bs, req, ctx, L, clamp=np.inf)
    assert np.array_equal(got, want)
    assert np.isinf(got[0, 49:]).all() and np.isfinite(got[0, :49]).all()      # row (b 0, j 0): ctx 49
    assert got[np.isfinite(got)].max() > 60000                                  # no clamp on this path


def test_mqa_logits_oracle_vs_row_store():
    """The flat prefill statement equals index_logits on 132-byte rows built from the same codes and scales (block
    size 1, identity block table) with positions below ks masked."""
    g = torch.Generator().manual_seed(4)
    N, M = 50, 5
    k = bf16_bits(torch.randn(N, 128, generator=g) * 2)
    rows = np.zeros((N, 132), dtype=np.uint8)
    ref.index_key_write(k, np.arange(N), rows)
    codes, scales = rows[:, :128], rows[:, 128:].copy().view(np.float32)[:, 0]
    q = torch.randn(M, 64, 128, generator=g).float().numpy()
    w = torch.rand(M, 64, generator=g).numpy()
    ks = np.array([0, 3, 10, 49, 20])
    ke = np.array([50, 4, 30, 50, 20])
    got = ref.mqa_logits(q, codes, scales, w, ks, ke)
    want = ref.index_logits(q, w, rows, np.arange(N, dtype=np.int32)[None, :], 1, np.zeros(M, dtype=np.int64), ke, N,
                            clamp=np.inf)
    for m in range(M):
        want[m, :ks[m]] = -np.inf
    assert np.array_equal(np.isinf(got), np.isinf(want))
    fin = np.isfinite(want)                            # float64, summation order of different matrix shapes
    assert np.allclose(got[fin], want[fin], rtol=1e-12, atol=0)
    assert np.isinf(got[4]).all()                      # empty range
