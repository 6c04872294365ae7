"""Pins of the CPU oracle (oracle/spmla_ref.py) against library routines, invariants and brute force, so that the
GPU parity tests compare against something independently checked. No GPU needed."""
import numpy as np
import pytest
import torch

from oracle import spmla_ref as ref
from oracle import cpu_port
from tests.helpers import bf16_bits, distinct_idx, make_pool_656, make_q


# ------------------------------------------------------------------------------------------------ e4m3 codec
def _torch_e4m3(f):
    return torch.from_numpy(np.ascontiguousarray(f, dtype=np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_e4m3_encoder_exhaustive_vs_torch():
    """the C restatement (nearest-value search) and torch agree on every fp32 with exponent field 117..136 (both
    signs: |x| in [2^-10, 2^10), every subnormal / normal e4m3 boundary and the 448 / 464 / 480 edges)."""
    from oracle import build as ob
    L = ob.load()
    n = 1 << 23
    buf = np.empty(n, dtype=np.uint8)
    for sign in (0, 0x80000000):
        for e in range(117, 137):
            start = sign | (e << 23)
            L.oracle_e4m3_encode_bits(start, n, buf.ctypes.data)
            f = (np.arange(n, dtype=np.uint64) + start).astype(np.uint32).view(np.float32)
            assert np.array_equal(buf, _torch_e4m3(f)), hex(start)


def test_e4m3_numpy_encoder_vs_torch():
    g = np.random.default_rng(0)
    bits = g.integers(0, 2 ** 32, 4_000_000, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    f = f[np.isfinite(f)]
    specials = np.array([0.0, -0.0, 448, -448, 464, 464.00003, 479.99, 480, 1e30, 2 ** -9, 2 ** -10, 3 * 2 ** -11,
                         1.5 * 2 ** -9, 2 ** -6, 2 ** -6 * 1.0625, 2 ** -7 * 1.0625, np.inf, -np.inf],
                        dtype=np.float32)
    for arr in (f, specials, (g.standard_normal(1_000_000) * 50).astype(np.float32)):
        a = ref.e4m3_encode(arr)
        b = _torch_e4m3(arr)
        fin = np.isfinite(arr)
        assert np.array_equal(a[fin], b[fin])
    assert ref.e4m3_encode(np.array([np.nan], np.float32))[0] & 0x7F == 0x7F


def test_e4m3_decode_vs_torch():
    c = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(c).view(torch.float8_e4m3fn).float().numpy()
    got = ref.e4m3_decode(c)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(got[~np.isnan(got)], want[~np.isnan(want)])


def test_library_host_encoder_matches_torch():
    """the e4m3 encoder the kernels use (spmla_common.h, also compiled for the host) against torch on a sample"""
    pytest.importorskip("ctypes")
    from arcagi2_flashnext_dots3_amd import _lib
    L = _lib.lib()
    if not hasattr(L, "spmla_host_e4m3_encode"):
        pytest.skip("no host encoder hook in this build")
    import ctypes
    f = (np.random.default_rng(1).standard_normal(1_000_000) * 100).astype(np.float32)
    out = np.empty(f.size, dtype=np.uint8)
    L.spmla_host_e4m3_encode(f.ctypes.data_as(ctypes.c_void_p), out.ctypes.data_as(ctypes.c_void_p),
                             ctypes.c_longlong(f.size))
    assert np.array_equal(out, _torch_e4m3(f))


# ------------------------------------------------------------------------------------------------ KV write
def _kv(n, seed):
    g = torch.Generator().manual_seed(seed)
    kv = torch.randn(n, 512, generator=g) * torch.exp(torch.randn(n, 1, generator=g) * 2)
    kv[0] = 0
    kv[1, 128:256] = 0
    pe = torch.randn(n, 64, generator=g)
    return bf16_bits(kv), bf16_bits(pe)


def test_cache_write_656_closed_form():
    n, R = 64, 100
    kv, pe = _kv(n, 0)
    slots = np.arange(n) * 3 % R
    slots[5] = -1
    cache = np.full((R, 656), 0x5A, dtype=np.uint8)
    ref.cache_write_656(kv, pe, slots, cache)
    x = ref.bf16_bits_to_f32(kv).reshape(n, 4, 128)
    for i in range(n):
        if slots[i] < 0:
            continue
        row = cache[slots[i]]
        s = row[512:528].copy().view(np.float32)
        codes = row[:512].reshape(4, 128)
        amax = np.abs(x[i]).max(-1)
        # scale closed form: max(amax / 448, 1e-12) in fp32
        assert np.array_equal(s, np.maximum((amax / np.float32(448)).astype(np.float32), np.float32(1e-12)))
        dq = ref.e4m3_decode(codes).astype(np.float64)
        y = (x[i] / s[:, None]).astype(np.float64)
        # every code is a nearest e4m3 value of x / s: error <= half the e4m3 spacing at that magnitude
        mag = np.maximum(np.abs(y), 2.0 ** -6)
        ulp = 2.0 ** (np.floor(np.log2(mag)) - 3)
        assert np.all(np.abs(dq - y) <= ulp / 2 + 1e-12)
        for g in range(4):
            if amax[g] > 0:
                k = np.argmax(np.abs(x[i, g]))
                assert codes[g, k] & 0x7F == 0x7E          # the group maximum encodes as +-448
            else:
                assert np.all(codes[g] == 0)
        assert np.array_equal(row[528:].view(np.uint16), pe[i])
    assert np.all(cache[[r for r in range(R) if r not in set(slots.tolist())]] == 0x5A)


def test_cache_write_576_clamps():
    kv = bf16_bits(torch.tensor([[1000.0, -1000.0, 1.0] + [0.0] * 509]))
    pe = bf16_bits(torch.zeros(1, 64))
    cache = np.zeros((1, 576), dtype=np.uint8)
    ref.cache_write_576(kv, pe, np.array([0]), cache, kv_scale=1.0)
    assert cache[0, 0] == 0x7E and cache[0, 1] == 0xFE and cache[0, 2] == 0x38


def test_index_key_write_closed_form():
    g = torch.Generator().manual_seed(3)
    k = bf16_bits(torch.randn(8, 128, generator=g) * 10)
    store = np.zeros((8, 132), dtype=np.uint8)
    ref.index_key_write(k, np.arange(8), store)
    x = ref.bf16_bits_to_f32(k)
    s = store[:, 128:].copy().view(np.float32)[:, 0]
    assert np.array_equal(s, (np.maximum(np.abs(x).max(1), np.float32(1e-4)) / np.float32(448)).astype(np.float32))
    store2 = np.zeros((8, 132), dtype=np.uint8)
    ref.index_key_write(k, np.arange(8), store2, ue8m0=True)
    s2 = store2[:, 128:].copy().view(np.float32)[:, 0]
    assert np.all(np.log2(s2) == np.round(np.log2(s2))) and np.all(s2 >= s) and np.all(s2 < 2 * s)


# ------------------------------------------------------------------------------------------------ attention
def _sdpa_ref(q, pool, idx, scale):
    """torch SDPA (float64) on dequantized rows with a boolean mask + torch.logsumexp"""
    lat, rope = ref.dequant_656(pool)
    rows = torch.from_numpy(np.concatenate([lat, rope], 1))
    T, H, _ = q.shape
    out = np.zeros((T, H, 512))
    lse = np.full((T, H), -np.inf)
    for t in range(T):
        sel = [int(i) for i in idx[t] if 0 <= i < pool.shape[0]]
        if not sel:
            continue
        k = rows[sel]
        qt = torch.from_numpy(q[t]).double()
        o = torch.nn.functional.scaled_dot_product_attention(qt[None, None], k[None, None], k[None, None, :, :512],
                                                             scale=scale)[0, 0]
        out[t] = o.numpy()
        lse[t] = torch.logsumexp(qt @ k.T * scale, dim=-1).numpy()
    return out, lse


def test_attention_oracle_vs_sdpa():
    pool, _, _ = make_pool_656(600, seed=4)
    q = make_q(3, 8, seed=5).float().numpy()
    idx = distinct_idx(3, 50, 600, seed=6).numpy()
    idx[1, 10:] = -1
    idx[2, :] = 700                 # all invalid
    o, l = ref.attention(q, pool, idx, 192 ** -0.5)
    o2, l2 = _sdpa_ref(q, pool, idx, 192 ** -0.5)
    assert np.allclose(o, o2, atol=1e-12) and np.array_equal(np.isinf(l), np.isinf(l2))
    assert np.allclose(l[np.isfinite(l)], l2[np.isfinite(l2)], atol=1e-12)
    assert np.all(o[2] == 0) and np.all(np.isneginf(l[2]))


def test_attention_brute_force_tiny():
    pool, _, _ = make_pool_656(20, seed=7)
    q = make_q(1, 2, seed=8).float().numpy()
    idx = np.array([[3, 7, 7, 19]])                      # duplicate counted twice
    o, l = ref.attention(q, pool, idx, 0.1)
    lat, rope = ref.dequant_656(pool)
    for h in range(2):
        s = [0.1 * sum(q[0, h, d] * (lat[r, d] if d < 512 else rope[r, d - 512]) for d in range(576))
             for r in idx[0]]
        m = max(s)
        e = [np.exp(v - m) for v in s]
        want = sum(e[k] * lat[idx[0, k]] for k in range(4)) / sum(e)
        assert np.allclose(o[0, h], want, atol=1e-10)
        assert abs(l[0, h] - (m + np.log(sum(e)))) < 1e-10


def test_attention_permutation_invariance_and_merge():
    pool, _, _ = make_pool_656(500, seed=9)
    q = make_q(2, 4, seed=10).float().numpy()
    idx = distinct_idx(2, 96, 500, seed=11).numpy()
    o, l = ref.attention(q, pool, idx, 0.07)
    perm = np.random.default_rng(0).permutation(96)
    o2, l2 = ref.attention(q, pool, idx[:, perm], 0.07)
    assert np.allclose(o, o2, atol=1e-12) and np.allclose(l, l2, atol=1e-12)
    parts = [ref.attention(q, pool, idx[:, a:b], 0.07) for a, b in ((0, 10), (10, 50), (50, 96))]
    om, lm = ref.lse_merge(np.stack([p[0] for p in parts]), np.stack([p[1] for p in parts]))
    assert np.allclose(om, o, atol=1e-12) and np.allclose(lm, l, atol=1e-12)
    # a part with no rows (-inf) leaves the merge unchanged; all parts empty -> 0 / -inf
    empty = (np.zeros_like(o), np.full_like(l, -np.inf))
    om2, lm2 = ref.lse_merge(np.stack([o, empty[0]]), np.stack([l, empty[1]]))
    assert np.allclose(om2, o) and np.allclose(lm2, l)
    om3, lm3 = ref.lse_merge(np.stack([empty[0]] * 2), np.stack([empty[1]] * 2))
    assert np.all(om3 == 0) and np.all(np.isneginf(lm3))


def test_cpu_port_matches_oracle():
    pool, _, _ = make_pool_656(3000, seed=12)
    q = make_q(4, 16, seed=13)
    idx = distinct_idx(4, 256, 3000, seed=14)
    o, l = cpu_port.attention_f32(q, torch.from_numpy(pool), idx, 192 ** -0.5)
    o2, l2 = ref.attention(q.float().numpy(), pool, idx.numpy(), 192 ** -0.5)
    assert np.abs(o.numpy() - o2).max() < 1e-4 and np.abs(l.numpy() - l2).max() < 1e-4


# ------------------------------------------------------------------------------------------------ indexer
def _store(n, seed):
    g = torch.Generator().manual_seed(seed)
    k = bf16_bits(torch.randn(n, 128, generator=g))
    st = np.zeros((n, 132), dtype=np.uint8)
    ref.index_key_write(k, np.arange(n), st)
    return st


def test_index_logits_brute_force_and_linearity():
    bs, L = 4, 10
    st = _store(16, 0)
    bt = np.array([[2, 0, 3], [1, 2, 0]], dtype=np.int64)
    g = np.random.default_rng(1)
    q = (g.standard_normal((2, 64, 128))).astype(np.float32)
    w = g.random((2, 64)).astype(np.float32)
    req = np.array([1, 0])
    ctx = np.array([10, 7])
    out = ref.index_logits(q, w, st, bt, bs, req, ctx, L)
    kc = ref.e4m3_decode(st[:, :128]).astype(np.float64)
    ks = st[:, 128:].copy().view(np.float32)[:, 0]
    for r in range(2):
        for j in range(L):
            if j >= ctx[r]:
                assert out[r, j] == -np.inf
                continue
            row = bt[req[r], j // bs] * bs + j % bs
            v = 0.0
            for h in range(64):
                v += float(w[r, h]) * max(0.0, float(np.dot(q[r, h].astype(np.float64), kc[row])))
            assert abs(out[r, j] - min(v * float(ks[row]), 60000.0)) < 1e-9 * max(1, abs(v))
    w2 = g.random((2, 64)).astype(np.float32)
    a = ref.index_logits(q, w, st, bt, bs, req, ctx, L, clamp=np.inf)
    b = ref.index_logits(q, w2, st, bt, bs, req, ctx, L, clamp=np.inf)
    c = ref.index_logits(q, w + w2, st, bt, bs, req, ctx, L, clamp=np.inf)
    fin = np.isfinite(a)
    assert np.allclose(a[fin] + b[fin], c[fin], rtol=1e-6)


def _topk_brute(row, n, K):
    items = [(float(v), j) for j, v in enumerate(row[:n])]
    key = lambda it: (ref.okey(np.float32(it[0])).item(), -it[1])
    items.sort(key=key, reverse=True)
    out = [(-1 if np.isinf(v) else j) for v, j in items[:K]]
    return out + [-1] * (K - len(out))


def test_topk_brute_force_ties_and_specials():
    g = np.random.default_rng(2)
    rows = [np.round(g.standard_normal(60) * 2) / 2, np.zeros(60), np.where(g.random(60) > .5, 0.0, -0.0),
            np.full(60, -np.inf), g.standard_normal(60)]
    rows[4][[3, 9]] = np.nan
    rows[4][5] = np.inf
    lg = np.stack(rows).astype(np.float32)
    ctx = np.array([60, 60, 60, 60, 33], dtype=np.int32)
    out = ref.topk(lg, ctx, 20)
    for r in range(len(rows)):
        assert out[r].tolist() == _topk_brute(lg[r], ctx[r], 20)


def test_topk_vs_torch_topk_sets():
    g = np.random.default_rng(3)
    lg = g.standard_normal((6, 5000)).astype(np.float32)
    ctx = np.array([5000, 4000, 2048, 2047, 100, 0], dtype=np.int32)
    out = ref.topk(lg, ctx, 2048)
    for r in range(6):
        n = min(ctx[r], 5000)
        if n == 0:
            assert np.all(out[r] == -1)
            continue
        v, i = torch.topk(torch.from_numpy(lg[r, :n]), min(2048, n))
        assert set(out[r][out[r] >= 0].tolist()) == set(i.tolist())
        assert np.all(np.diff(lg[r, out[r][out[r] >= 0]]) <= 0)


# ------------------------------------------------------------------------------------------------ rows
def test_compact_stage_vs_torch_unique():
    g = np.random.default_rng(4)
    rows = g.integers(0, 10 ** 6, 300)
    sidx = g.integers(-1, 300, (7, 40)).astype(np.int32)
    sel, s2 = ref.compact_stage(rows, sidx)
    t = torch.from_numpy(sidx.astype(np.int64))
    v = t >= 0
    u, inv = torch.unique(t[v], sorted=True, return_inverse=True)
    assert np.array_equal(sel, rows[u.numpy()])
    want = np.full(sidx.shape, -1)
    want[v.numpy()] = inv.numpy()
    assert np.array_equal(s2, want)
    assert np.array_equal(np.where(sidx >= 0, rows[np.maximum(sidx, 0)], -1), np.where(s2 >= 0, sel[np.maximum(s2, 0)], -1))


def test_rows_from_topk_hand_example():
    bt = np.array([[5, -1, 2], [0, 7, 1]])
    topk = np.array([[0, 63, 64, 130, -1, 200], [65, 1, 192, 128, 3, 10]])
    req = np.array([0, 1])
    out = ref.rows_from_topk(topk, req, bt, 64)
    assert out.tolist() == [[320, 383, -1, 130, -1, -1], [449, 1, -1, 64, 3, 10]]


def test_tier_split_and_gather_hand_example():
    rowmap = np.array([-1, 0, -1, 1, -1], dtype=np.int32)
    hbm, hc, host, sc = ref.tier_split(np.array([[3, 0, 1, -1, 2, 9, 3]]), rowmap, 5)
    assert hbm[0, :3].tolist() == [1, 0, 1] and hc[0] == 3 and np.all(hbm[0, 3:] == -1)
    assert host[0, :2].tolist() == [0, 2] and sc[0] == 2 and np.all(host[0, 2:] == -1)
    src = np.arange(12, dtype=np.uint8).reshape(3, 4)
    assert ref.gather(src, np.array([2, -1, 0, 3])).tolist() == [[8, 9, 10, 11], [0] * 4, [0, 1, 2, 3], [0] * 4]


def test_topk_fp16_order_is_the_widened_fp32_order():
    """The oracle selects on fp16 logits by widening them to fp32: over all 65536 fp16 patterns, the fp32 order key
    of the widened value orders and ties them exactly as python's float comparison does (NaN largest, -0 below +0),
    i.e. as the reference's 16-bit key does."""
    import functools
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = h.view(np.float16).astype(np.float64)

    def cmp(a, b):                                  # NaN largest, then value, then -0 < +0
        na, nb = np.isnan(f[a]), np.isnan(f[b])
        if na or nb:
            return int(na) - int(nb)
        if f[a] != f[b]:
            return -1 if f[a] < f[b] else 1
        sa, sb = np.signbit(f[a]), np.signbit(f[b])
        return int(sb) - int(sa)
    k = ref.okey(h.view(np.float16).astype(np.float32)).astype(np.int64)
    g = np.random.default_rng(9)
    a, b = g.integers(0, 65536, 20000), g.integers(0, 65536, 20000)
    for x, y in zip(a, b):
        c = cmp(x, y)
        assert (k[x] < k[y]) == (c < 0 and not (np.isnan(f[x]) and np.isnan(f[y])))
        assert (k[x] == k[y]) == (c == 0 or (np.isnan(f[x]) and np.isnan(f[y])))
    srt = sorted(range(0, 65536, 7), key=functools.cmp_to_key(cmp))
    assert (np.diff(k[srt]) >= 0).all()
    # the widened row gives the same selection as brute force on the fp16 values
    row = g.standard_normal(300).astype(np.float16)
    row[::7] = 0.5
    row[3] = np.float16(-0.0)
    exp = sorted(range(300), key=lambda j: (-float(row[j]), j))[:64]
    assert list(ref.topk(row[None].astype(np.float32), np.array([300]), 64)[0]) == exp
