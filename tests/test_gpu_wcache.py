"""GPU checks of the dynamic W-way row cache (spmla_wcache_*) against the oracle's order-independent model of a cache
step (hits, misses, spills, pinned lines kept, the lines that receive misses, set contents where no set overflows,
round-robin pointers), the bytes every entry resolves to, and attention through the cache vs a single-tier pass."""
import numpy as np
import pytest
import torch

from oracle import spmla_ref as ref
from tests.helpers import attn_excess, make_pool_656, make_q

pytestmark = pytest.mark.gpu


def _selections(T, K, R, step, hot=600):
    """Skewed selections: half the entries from a small hot range (so later steps hit), the rest uniform, some
    invalid entries."""
    g = np.random.default_rng(100 + step)
    a = g.integers(0, hot, (T, K))
    b = g.integers(0, R, (T, K))
    idx = np.where(g.random((T, K)) < 0.5, a, b)
    idx[:, ::97] = -1
    idx[0, 5] = R + 3
    return idx.astype(np.int32)


def _check_step(wc, host_rows, idx, res, tag0, rr0, R):
    W, C, S = wc.W, wc.C, wc.S
    m = ref.wcache_step(tag0, rr0, idx, R, W)
    st = wc.state.cpu().numpy()
    assert st[3] == m["hits"] and st[1] == len(m["misses"]) and st[2] == m["spills"], (st, m["hits"], m["spills"])
    tag = wc.tag.cpu().numpy().astype(np.int64)
    assert np.array_equal(wc.rr.cpu().numpy(), m["rr_next"])
    for l in m["pinned"]:
        assert tag[l] == tag0[l]
    placed = {l for v in m["placed"].values() for l in v}
    changed = set(np.nonzero(tag != tag0)[0].tolist())
    assert changed <= placed and all(tag[l] in set(m["misses"]) for l in placed)
    for s_, want in m["content"].items():
        assert sorted(tag[s_ * W:(s_ + 1) * W].tolist()) == want
    for s_ in range(S):                                    # each row in its own set, at most once
        v = [x for x in tag[s_ * W:(s_ + 1) * W] if x >= 0]
        assert len(v) == len(set(v)) and all(x % S == s_ for x in v)
    pool = wc.pool.cpu().numpy()
    res = res.cpu().numpy()
    valid = (idx >= 0) & (idx < R)
    assert np.all(res[~valid] == -1) and np.all(res[valid] >= 0)
    rr_ = res[valid]
    assert np.array_equal(pool[rr_], host_rows[idx[valid]])
    line = rr_ < C
    assert np.all(tag[rr_[line]] == idx[valid][line])    # a line entry's tag is its row
    sp = {}
    for r, h in zip(rr_[~line], idx[valid][~line]):      # one spill row per distinct row
        assert sp.setdefault(h, r) == r
    assert len(set(sp.values())) == len(sp)


@pytest.mark.parametrize("W,host_fmt,pool_fmt", [(4, 0, 0), (16, 0, 0), (16, 2, 0), (8, 2, 2)])
def test_wcache_steps(dev, W, host_fmt, pool_fmt):
    """pool_fmt 2: compact Row400 lines, which receive the host's Row400 bytes as they are."""
    from arcagi2_flashnext_dots3_amd import kernels
    R, C, T, K = 20000, 1024, 4, 512
    if host_fmt == 0:
        host_np, _, _ = make_pool_656(R, seed=3)
        host_rows = host_np
    else:
        g = torch.Generator().manual_seed(3)
        kv = ref.f32_to_bf16_bits(torch.randn(R, 512, generator=g).numpy())
        pe = ref.f32_to_bf16_bits(torch.randn(R, 64, generator=g).numpy())
        host_np = np.zeros((R, 400), dtype=np.uint8)
        ref.cache_write_400(kv, pe, np.arange(R), host_np)
        host_rows = host_np if pool_fmt == 2 else ref.row400_gather(host_np, np.arange(R), fmt=656)
    host = torch.from_numpy(host_np).pin_memory()
    wc = kernels.RowCache(C, W, T * K, dev, row_bytes=400 if pool_fmt == 2 else 656)
    for step in range(6):
        idx = _selections(T, K, R, step)
        tag0, rr0 = wc.tag.cpu().numpy().astype(np.int64), wc.rr.cpu().numpy()
        print(f"[wcache] W={W} fmt={host_fmt} step={step}", flush=True)
        res = kernels.wcache_step(wc, torch.from_numpy(idx).to(dev), R)
        hit, hc, fresh, fc = kernels.wcache_split(wc, res)
        kernels.wcache_fill(wc, host, R, host_fmt, T * K)
        torch.cuda.synchronize()
        _check_step(wc, host_rows, idx, res, tag0, rr0, R)
        # hits: entries whose row was in its set before the step, in order; fresh: the other valid entries
        r = res.cpu().numpy()
        S = wc.S
        was = np.array([[0 <= h < R and h in set(tag0[(h % S) * W:(h % S + 1) * W].tolist()) for h in row]
                        for row in idx])
        valid = (idx >= 0) & (idx < R)
        hit, hc, fresh, fc = [x.cpu().numpy() for x in (hit, hc, fresh, fc)]
        for t in range(T):
            assert np.array_equal(hit[t, :hc[t]], r[t][was[t]]) and np.all(hit[t, hc[t]:] == -1)
            assert np.array_equal(fresh[t, :fc[t]], r[t][valid[t] & ~was[t]]) and np.all(fresh[t, fc[t]:] == -1)
    assert int(wc.state[3]) > 0                            # later steps hit the hot range


def test_wcache_overflow_and_invalidate(dev):
    """A cache far smaller than a step's misses: overfull sets spill (cap rows), the rest stay on the host (-2);
    invalidated rows miss at the next step and are served from their rewritten host rows."""
    from arcagi2_flashnext_dots3_amd import kernels
    R, C, W, T, K, cap = 5000, 64, 4, 2, 400, 100
    host_np, _, _ = make_pool_656(R, seed=4)
    host = torch.from_numpy(host_np).pin_memory()
    wc = kernels.RowCache(C, W, cap, dev)
    idx = np.random.default_rng(1).integers(0, R, (T, K)).astype(np.int32)
    tag0, rr0 = wc.tag.cpu().numpy().astype(np.int64), wc.rr.cpu().numpy()
    res = kernels.wcache_step(wc, torch.from_numpy(idx).to(dev), R)
    kernels.wcache_fill(wc, host, R, 0, T * K)
    torch.cuda.synchronize()
    m = ref.wcache_step(tag0, rr0, idx, R, W)
    st = wc.state.cpu().numpy()
    assert st[2] == m["spills"] and m["spills"] > cap
    r = res.cpu().numpy()
    pool = wc.pool.cpu().numpy()
    assert np.all(r >= -2) and (r == -2).sum() > 0
    ok = r >= 0
    assert np.array_equal(pool[r[ok]], host_np[idx[ok]])
    # host tier split: every -2 entry appears on the host list in order
    hb, hc, hs, sc = kernels.split_res(torch.from_numpy(idx).to(dev), res)
    hb, hc, hs, sc = [x.cpu().numpy() for x in (hb, hc, hs, sc)]
    for t in range(T):
        assert np.array_equal(hb[t, :hc[t]], r[t][r[t] >= 0]) and np.all(hb[t, hc[t]:] == -1)
        assert np.array_equal(hs[t, :sc[t]], idx[t][r[t] == -2]) and np.all(hs[t, sc[t]:] == -1)
    # invalidate the cached rows of token 0 and check that the next step misses them
    cached = np.array(sorted({int(h) for h in idx[0] if h in set(wc.tag.cpu().numpy().tolist())}), dtype=np.int64)
    assert cached.size
    kernels.wcache_invalidate(wc, torch.from_numpy(cached).to(dev), R)
    torch.cuda.synchronize()
    assert not np.isin(wc.tag.cpu().numpy(), cached).any()


@pytest.mark.parametrize("cap,overlap", [(4096, False), (4096, True), (64, True)])
def test_layer_offload_ways_matches_single_tier(dev, cap, overlap):
    """LayerOffload(cache_mode='ways') over several steps: with a spill area covering the step and no overlap, the
    attention over the cache pool equals the single-tier attention over the gathered rows bit for bit (same row bytes,
    same order); with the hits attended beside the copy, or a small spill area that leaves rows on the host, the
    merged result matches within the tier-merge tolerance."""
    from arcagi2_flashnext_dots3_amd import kernels
    from arcagi2_flashnext_dots3_amd.sparse_offload import LayerOffload
    R, T, H, K = 6000, 4, 64, 1024
    g = torch.Generator().manual_seed(5)
    kv = (torch.randn(R, 512, generator=g)).to(torch.bfloat16)
    pe = torch.randn(R, 64, generator=g).to(torch.bfloat16)
    lo = LayerOffload(R, dev, cache_rows=512, cache_mode="ways", ways=8, spill_rows=cap, overlap_fill=overlap)
    lo.store(kv.to(dev), pe.to(dev), torch.arange(R, dtype=torch.int64, device=dev))
    q = make_q(T, H, seed=6).to(dev)
    sm = 192 ** -0.5
    for step in range(4):
        idx = torch.from_numpy(_selections(T, K, R, step, hot=300)).to(dev)
        out, lse = lo.attend(q, idx, sm, return_lse=True)
        staged = torch.empty(T * K, 656, dtype=torch.uint8, device=dev)
        kernels.gather(lo.host, idx.reshape(-1).to(torch.int64), staged)
        sidx = torch.where((idx >= 0) & (idx < R), torch.arange(T * K, device=dev, dtype=torch.int32).view(T, K),
                           torch.full_like(idx, -1))
        o1, l1 = kernels.attend(q, staged, sidx, sm)
        torch.cuda.synchronize()
        if cap >= T * K and not overlap:
            assert torch.equal(out, o1) and torch.equal(lse, l1)
        else:
            # both sides are bf16 outputs rounded separately: each within 1e-2 of the fp32 result can still differ
            # from the other by one bf16 ulp, 2^-6 > 1e-2 for |x| in [2, 4); the bound is 1e-2 * max(1, |x|)
            err = (out.float() - o1.float()).abs() / o1.float().abs().clamp_min(1.0)
            assert float(err.max()) <= 1e-2
            assert float((lse - l1).abs().max()) <= 1e-4
    assert lo.hit_rate(idx) > 0.0


@pytest.mark.parametrize("W,cap", [(1, 4096), (4, 4096), (4, 48)])
def test_wcache_two_choice_steps(dev, W, cap):
    """Two-choice placement over several steps of a cache much smaller than the working set (sets overflow): hits,
    distinct misses and every outcome condition of the oracle's verifier (pinned lines kept, rows only in their two
    sets and at most once, first-p unpinned ways per set, p = min(tickets, free), full sets before a second-set or
    spill placement, rr advance); every entry's pool row holds its host row; invalidation clears both sets."""
    from arcagi2_flashnext_dots3_amd import kernels
    R, C, T, K = 6000, 256, 4, 256
    host_np, _, _ = make_pool_656(R, seed=8)
    host = torch.from_numpy(host_np).pin_memory()
    wc = kernels.RowCache(C, W, cap, dev, two=True)
    S = wc.S
    second = 0
    for step in range(5):
        idx = _selections(T, K, R, step, hot=400)
        tag0, rr0 = wc.tag.cpu().numpy().astype(np.int64), wc.rr.cpu().numpy()
        print(f"[wcache two] W={W} cap={cap} step={step}", flush=True)
        res = kernels.wcache_step(wc, torch.from_numpy(idx).to(dev), R)
        kernels.wcache_fill(wc, host, R, 0, T * K)
        torch.cuda.synchronize()
        m = ref.wcache_step2(tag0, rr0, idx, R, W)
        st = wc.state.cpu().numpy()
        assert st[3] == m["hits"] and st[1] == len(m["misses"]), (st, m["hits"], len(m["misses"]))
        tag = wc.tag.cpu().numpy().astype(np.int64)
        bad = ref.wcache_verify2(m, tag0, rr0, tag, wc.rr.cpu().numpy(), int(st[2]))
        assert bad == [], bad[:5]
        second += sum(1 for l in np.nonzero(tag != tag0)[0] if l // W != tag[l] % S)
        r = res.cpu().numpy()
        valid = (idx >= 0) & (idx < R)
        assert np.all(r[~valid] == -1) and np.all(r[valid] >= -2)
        ok = r >= 0
        pool = wc.pool.cpu().numpy()
        assert np.array_equal(pool[r[ok]], host_np[idx[ok]])
        line = ok & (r < C)
        assert np.all(tag[r[line]] == idx[line])
        if cap >= T * K:
            assert np.all(r[valid] >= 0)
    assert second > 0                                      # some misses took their second set
    cached = np.unique(tag[tag >= 0])
    kernels.wcache_invalidate(wc, torch.from_numpy(cached.astype(np.int64)).to(dev), R)
    torch.cuda.synchronize()
    assert np.all(wc.tag.cpu().numpy() == -1)


def test_layer_offload_two_choice_matches_single_tier(dev):
    """LayerOffload(cache_mode='ways', two_choice=True) with a spill area covering the step and no overlap: the
    attention over the cache pool equals the single-tier attention over the gathered rows bit for bit."""
    from arcagi2_flashnext_dots3_amd import kernels
    from arcagi2_flashnext_dots3_amd.sparse_offload import LayerOffload
    R, T, H, K = 6000, 4, 64, 1024
    g = torch.Generator().manual_seed(9)
    kv = (torch.randn(R, 512, generator=g)).to(torch.bfloat16)
    pe = torch.randn(R, 64, generator=g).to(torch.bfloat16)
    lo = LayerOffload(R, dev, cache_rows=512, cache_mode="ways", ways=8, spill_rows=T * K, overlap_fill=False,
                      two_choice=True)
    lo.store(kv.to(dev), pe.to(dev), torch.arange(R, dtype=torch.int64, device=dev))
    q = make_q(T, H, seed=10).to(dev)
    sm = 192 ** -0.5
    for step in range(3):
        idx = torch.from_numpy(_selections(T, K, R, step, hot=300)).to(dev)
        out, lse = lo.attend(q, idx, sm, return_lse=True)
        staged = torch.empty(T * K, 656, dtype=torch.uint8, device=dev)
        kernels.gather(lo.host, idx.reshape(-1).to(torch.int64), staged)
        sidx = torch.where((idx >= 0) & (idx < R), torch.arange(T * K, device=dev, dtype=torch.int32).view(T, K),
                           torch.full_like(idx, -1))
        o1, l1 = kernels.attend(q, staged, sidx, sm)
        torch.cuda.synchronize()
        assert torch.equal(out, o1) and torch.equal(lse, l1)
    assert lo.hit_rate(idx) > 0.0


@pytest.mark.parametrize("cap,overlap", [(4096, False), (4096, True), (64, True)])
def test_layer_offload_compact_ways(dev, cap, overlap):
    """The reference's production offload mode (mode_submit.json: ARC_OFFLOAD_WAYS=8, ARC_OFFLOAD_ROW_FMT=e2m2,
    ARC_OFFLOAD_CCACHE=1, ARC_OFFLOAD_OVERLAP=1, ARC_OFFLOAD_TWO_CHOICE=1): compact Row400 host rows and compact
    Row400 lines in an 8-way two-choice pool, the step's pool rows decoded for the attention. With a spill area
    covering the step and no overlap, the result equals bit for bit the single-tier attention over the host rows
    decoded to Row576 (same bytes, same kernel, same order); with the overlap or a small spill area (rows left on the
    host) it matches within the tier-merge tolerance; and it matches the fp64 oracle over the decoded rows."""
    from arcagi2_flashnext_dots3_amd import kernels
    from arcagi2_flashnext_dots3_amd.sparse_offload import LayerOffload
    R, T, H, K, ks = 6000, 4, 64, 1024, 0.5
    g = torch.Generator().manual_seed(11)
    kv = (torch.randn(R, 512, generator=g) * 2).to(torch.bfloat16)
    pe = torch.randn(R, 64, generator=g).to(torch.bfloat16)
    lo = LayerOffload(R, dev, cache_rows=512, cache_mode="ways", ways=8, spill_rows=cap, overlap_fill=overlap,
                      two_choice=True, row_fmt="e2m2", cache_fmt="e2m2")
    assert lo.wc.pool.shape[1] == 400
    lo.store(kv.to(dev), pe.to(dev), torch.arange(R, dtype=torch.int64, device=dev), kv_scale=ks)
    q = make_q(T, H, seed=12).to(dev)
    sm = 192 ** -0.5
    host_np = lo.host.numpy()
    for step in range(4):
        print(f"[compact ways] cap={cap} overlap={overlap} step={step}", flush=True)
        idx = torch.from_numpy(_selections(T, K, R, step, hot=300)).to(dev)
        out, lse = lo.attend(q, idx, sm, ks, return_lse=True)
        staged = torch.empty(T * K, 576, dtype=torch.uint8, device=dev)
        kernels.row400_gather(lo.host, idx.reshape(-1).to(torch.int64), staged, pcie=True)
        sidx = torch.where((idx >= 0) & (idx < R), torch.arange(T * K, device=dev, dtype=torch.int32).view(T, K),
                           torch.full_like(idx, -1))
        o1, l1 = kernels.attend(q, staged, sidx, sm, ks)
        torch.cuda.synchronize()
        if cap >= T * K and not overlap:
            assert torch.equal(out, o1) and torch.equal(lse, l1)
        else:
            err = (out.float() - o1.float()).abs() / o1.float().abs().clamp_min(1.0)
            assert float(err.max()) <= 1e-2
            assert float((lse - l1).abs().max()) <= 1e-4
        if step == 3:
            i_np = idx.cpu().numpy()
            rows576 = ref.row400_gather(host_np, i_np.reshape(-1), fmt=576)
            local = np.where((i_np >= 0) & (i_np < R), np.arange(T * K).reshape(T, K), -1)
            eo, el = ref.attention(q.float().cpu().numpy(), rows576, local, sm, ks, fmt=576)
            assert attn_excess(out.float().cpu().numpy(), eo) <= 0
            fin = np.isfinite(el)
            assert np.abs(lse.cpu().numpy()[fin] - el[fin]).max() <= 1e-3
    st = lo.wc.state.cpu().numpy()
    assert lo.hit_rate(idx) > 0.0 and st[3] > 0
