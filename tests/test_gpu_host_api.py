"""GPU parity of the host-side mirror of the reference's interfaces: fast_topk.local / merge, ShardStore +
sharded_topk, LayerOffload (store / gather / tiered attend) and PortableSparseImpl (paged and offload paths), each
checked against the oracle on the same seeded inputs."""
import numpy as np
import pytest
import torch

from oracle import spmla_ref as ref
from tests.helpers import attn_excess, bf16_bits, distinct_idx, make_q

pytestmark = pytest.mark.gpu
SM = 192 ** -0.5


def _logits_rows(rows, L, seed, ties=False):
    g = np.random.RandomState(seed)
    lg = g.randn(rows, L).astype(np.float32)
    if ties:
        lg = np.round(lg * 4) / 4          # many exactly equal values
        lg[0, : L // 3] = 0.5
        lg[-1, 5] = -0.0
        lg[-1, 6] = 0.0
        lg[-1, 7] = np.inf
        lg[-1, 8] = -np.inf
        lg[-1, 9] = np.nan
    return lg


def _attn_err(o, lse, eo, el):
    """(excess of |o - eo| over 1e-2 + half a bf16 ulp of eo (passes when <= 0), max |lse - el|)."""
    fin = np.isfinite(el)
    assert np.array_equal(fin, np.isfinite(lse))
    e_l = np.max(np.abs(lse[fin] - el[fin])) if fin.any() else 0.0
    return attn_excess(o, eo), e_l


def _gpu_diff(o, lse, o1, l1):
    """(max |o - o1| / max(1, |o1|), max |lse - l1|) between two GPU results of the same attention."""
    fin = np.isfinite(l1)
    assert np.array_equal(fin, np.isfinite(lse))
    return np.max(np.abs(o - o1) / np.maximum(1.0, np.abs(o1))), (np.max(np.abs(lse[fin] - l1[fin])) if fin.any() else 0.0)


@pytest.mark.parametrize("rows,L,kl,ties", [(6, 3000, 256, False), (5, 1500, 512, True), (3, 100, 256, False)])
def test_topk_local_merge_p1(dev, rows, L, kl, ties):
    from arcagi2_flashnext_dots3_amd import fast_topk
    lg = _logits_rows(rows, L, rows + L, ties)
    ctx = np.array([L - 7 * i for i in range(rows)], dtype=np.int32)
    ctx[-1] = min(L, kl // 2)                      # a row with fewer valid columns than kl
    print(f"[local] rows={rows} L={L} kl={kl} ties={ties}", flush=True)
    pk = fast_topk.local(torch.from_numpy(lg).to(dev), torch.from_numpy(ctx).to(dev), 0, 1, kl)
    out = torch.full((rows, kl + 5), 7, dtype=torch.int32, device=dev)
    fast_topk.merge(pk, rows, 1, kl, kl, out)
    torch.cuda.synchronize()
    epk = ref.topk_local(lg, ctx, 0, 1, kl)
    assert np.array_equal(pk.cpu().numpy().view(np.uint32), epk.view(np.uint32))
    eo = ref.topk_merge(epk, rows, 1, kl, kl, kl + 5)
    assert np.array_equal(out.cpu().numpy(), eo)
    assert np.array_equal(eo[:, :kl], ref.topk(lg, ctx, kl))   # local + merge == one exact top-k at P = 1


def test_topk_local_merge_p2(dev):
    """Two ranks' shards of one logits row (position j * 2 + rank), local select per rank, rank-major merge."""
    from arcagi2_flashnext_dots3_amd import fast_topk
    rows, L, kl, kk = 4, 4000, 300, 512
    full = _logits_rows(rows, L, 11, ties=True)
    ctx = np.array([L, L - 1, 2001, 17], dtype=np.int32)
    pks, epks = [], []
    for rank in range(2):
        sh = np.ascontiguousarray(full[:, rank::2])
        pks.append(fast_topk.local(torch.from_numpy(sh).to(dev), torch.from_numpy(ctx).to(dev), rank, 2, kl))
        epks.append(ref.topk_local(sh, ctx, rank, 2, kl))
    allp = torch.cat(pks, 0).contiguous()
    out = torch.empty(rows, kk, dtype=torch.int32, device=dev)
    fast_topk.merge(allp, rows, 2, kl, kk, out)
    torch.cuda.synchronize()
    for r in range(2):
        assert np.array_equal(pks[r].cpu().numpy().view(np.uint32), epks[r].view(np.uint32))
    assert np.array_equal(out.cpu().numpy(), ref.topk_merge(np.concatenate(epks, 0), rows, 2, kl, kk, kk))


def test_shard_store_and_sharded_topk(dev):
    from arcagi2_flashnext_dots3_amd import shard_indexer
    rows, bs, nb, L, K = 3, 64, 160, 3000, 512
    g = torch.Generator().manual_seed(5)
    kc = torch.zeros(nb, bs, 132, dtype=torch.uint8, device=dev)
    st = shard_indexer.ShardStore(kc, 1, 0)
    k = torch.randn(nb * bs, 128, generator=g).to(torch.bfloat16)
    slots = torch.randperm(nb * bs, generator=g)[: nb * bs - 100]
    st.write(k.to(dev), slots.to(dev), False)
    torch.cuda.synchronize()
    store = np.zeros((nb * bs, 132), dtype=np.uint8)
    ref.index_key_write(bf16_bits(k), slots.numpy(), store)
    assert np.array_equal(kc.cpu().numpy().reshape(-1, 132), store)
    nbp = (L + bs - 1) // bs
    bt = torch.randperm(nb, generator=g)[: rows * nbp].reshape(rows, nbp).to(torch.int32)
    q = torch.randn(rows, 64, 128, generator=g).to(torch.bfloat16)
    w = torch.rand(rows, 64, generator=g)
    req = torch.arange(rows, dtype=torch.int32)
    ctx = torch.tensor([L, 1777, 300], dtype=torch.int32)
    lg = st.logits(q.to(dev), w.to(dev), bt.to(dev), req.to(dev), ctx.to(dev), L)
    out = torch.empty(rows, K + 3, dtype=torch.int32, device=dev)
    shard_indexer.sharded_topk(st, q.to(dev), w.to(dev), bt.to(dev), req.to(dev), ctx.to(dev), L, out, K + 3)
    torch.cuda.synchronize()
    glg = lg.cpu().numpy()
    exp_lg = ref.index_logits(q.float().numpy(), w.numpy(), store, bt.numpy(), bs, req.numpy(), ctx.numpy(), L)
    fin = np.isfinite(exp_lg)
    assert np.array_equal(np.isinf(glg), np.isinf(exp_lg))
    assert np.max(np.abs(glg[fin] - exp_lg[fin]) / np.maximum(1, np.abs(exp_lg[fin]))) <= 2e-5
    # selection is exact on the GPU's own logits
    assert np.array_equal(out.cpu().numpy(), ref.topk(glg, ctx.numpy(), K + 3))
    # the reference's fp8 indexer query (shard_indexer.py:118-120): e4m3 queries give the logits of their exact bf16
    # values, bit for bit, and the fp64 oracle's over those values
    q8 = (q.float() * 4.0).to(torch.float8_e4m3fn)
    lg8 = st.logits(q8.to(dev), w.to(dev), bt.to(dev), req.to(dev), ctx.to(dev), L)
    lgw = st.logits(q8.to(torch.bfloat16).to(dev), w.to(dev), bt.to(dev), req.to(dev), ctx.to(dev), L)
    torch.cuda.synchronize()
    assert torch.equal(lg8, lgw)
    exp8 = ref.index_logits(q8.float().numpy(), w.numpy(), store, bt.numpy(), bs, req.numpy(), ctx.numpy(), L)
    g8 = lg8.cpu().numpy()
    assert np.array_equal(np.isinf(g8), np.isinf(exp8))
    assert np.max(np.abs(g8[fin] - exp8[fin]) / np.maximum(1, np.abs(exp8[fin]))) <= 2e-5


def _offload_layer(dev, R, C, seed, **kw):
    from arcagi2_flashnext_dots3_amd.sparse_offload import LayerOffload
    g = torch.Generator().manual_seed(seed)
    kv = torch.randn(R, 512, generator=g).to(torch.bfloat16)
    pe = torch.randn(R, 1, 64, generator=g).to(torch.bfloat16)
    lo = LayerOffload(R, dev, key="model.layers.3.self_attn.indexer.k_cache", cache_rows=C, **kw)
    slots = torch.randperm(R, generator=g)
    lo.store(kv.to(dev), pe.to(dev), slots.to(dev))
    torch.cuda.synchronize()
    pool = np.zeros((R, 656), dtype=np.uint8)
    ref.cache_write_656(bf16_bits(kv), bf16_bits(pe.reshape(R, 64)), slots.numpy(), pool)
    return lo, pool


def test_offload_store_gather_and_hot_rows(dev):
    from arcagi2_flashnext_dots3_amd.sparse_offload import hot_rows_by_frequency
    R, C = 3000, 700
    lo, pool = _offload_layer(dev, R, C, 3)
    assert np.array_equal(lo.host.numpy(), pool)
    rows = torch.tensor([5, -1, 2999, 3000, 17], dtype=torch.int64, device=dev)
    out = torch.full((5, 656), 9, dtype=torch.uint8, device=dev)
    lo.gather(rows, out)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), ref.gather(pool, rows.cpu().numpy()))
    counts = torch.zeros(R, dtype=torch.int64, device=dev)
    counts[torch.arange(0, R, 3, device=dev)] = torch.arange(0, R, 3, device=dev) % 7 + 1
    hot = hot_rows_by_frequency(counts, C)
    lo.set_hot_rows(hot)
    torch.cuda.synchronize()
    hot_np = hot.cpu().numpy()
    assert np.array_equal(lo.cache[: hot_np.size].cpu().numpy(), pool[hot_np])
    assert np.array_equal(lo.tag[: hot_np.size].cpu().numpy(), hot_np)
    # write-through: rewriting hot rows updates both tiers identically
    g = torch.Generator().manual_seed(9)
    kv = torch.randn(50, 512, generator=g).to(torch.bfloat16)
    pe = torch.randn(50, 64, generator=g).to(torch.bfloat16)
    slots = torch.from_numpy(np.concatenate([hot_np[:25], np.arange(1, 3000, 3)[:25]])).to(torch.int64)
    lo.store(kv.to(dev), pe.to(dev), slots.to(dev))
    torch.cuda.synchronize()
    ref.cache_write_656(bf16_bits(kv), bf16_bits(pe), slots.numpy(), pool)
    assert np.array_equal(lo.host.numpy(), pool)
    assert np.array_equal(lo.cache[: hot_np.size].cpu().numpy(), pool[hot_np])


@pytest.mark.parametrize("C", [0, 1500])
def test_offload_attend_tiers(dev, C):
    """Tiered attention (HBM hits + host misses, merged) equals single-pass attention over the same rows."""
    R, T, H, K = 4000, 3, 64, 512
    lo, pool = _offload_layer(dev, R, C, 4)
    if C:
        lo.set_hot_rows(torch.arange(0, 2 * C, 2, dtype=torch.int64, device=dev))
    q = make_q(T, H, seed=4)
    idx = distinct_idx(T, K, R, seed=5)
    idx[1, 100:] = -1                       # a short row
    idx[2, :] = torch.arange(0, 2 * K, 2)   # all hits when cached
    print(f"[offload attend] C={C} hit={lo.hit_rate(idx.to(dev)):.3f}", flush=True)
    o, lse = lo.attend(q.to(dev), idx.to(dev), SM, 1.0, H, return_lse=True)
    torch.cuda.synchronize()
    eo, el = ref.attention(q.float().numpy(), pool, idx.numpy(), SM)
    e_o, e_l = _attn_err(o.float().cpu().numpy(), lse.cpu().numpy(), eo, el)
    print(f"[offload attend] err o {e_o:.2e} lse {e_l:.2e}", flush=True)
    assert e_o <= 0 and e_l <= 1e-3


def test_offload_attend_host_direct(dev):
    """host_direct=True: the host-tier attention reads the pinned rows in place over PCIe (no staging copy), its
    partial merged with the HBM tier's; vs the fp64 oracle and vs the staged path of the same rows."""
    R, C, T, H, K = 4000, 1500, 3, 64, 512
    lo, pool = _offload_layer(dev, R, C, 4, host_direct=True)
    lo.set_hot_rows(torch.arange(0, 2 * C, 2, dtype=torch.int64, device=dev))
    q = make_q(T, H, seed=4)
    idx = distinct_idx(T, K, R, seed=5)
    idx[1, 100:] = -1                       # a short row
    idx[2, :] = torch.arange(0, 2 * K, 2)   # all hits
    print("[offload host direct]", flush=True)
    o, lse = lo.attend(q.to(dev), idx.to(dev), SM, 1.0, H, return_lse=True)
    lo.host_direct = False
    o2, l2 = lo.attend(q.to(dev), idx.to(dev), SM, 1.0, H, return_lse=True)
    torch.cuda.synchronize()
    eo, el = ref.attention(q.float().numpy(), pool, idx.numpy(), SM)
    e_o, e_l = _attn_err(o.float().cpu().numpy(), lse.cpu().numpy(), eo, el)
    print(f"[offload host direct] excess {e_o:.2e} lse {e_l:.2e}", flush=True)
    assert e_o <= 0 and e_l <= 1e-3
    d_o, d_l = _gpu_diff(o.float().cpu().numpy(), lse.cpu().numpy(), o2.float().cpu().numpy(), l2.cpu().numpy())
    assert d_o <= 1e-2 and d_l <= 1e-5


@pytest.mark.parametrize("C", [0, 1500])
def test_offload_attend_packed_mtp(dev, C):
    """packed=True with ql = 4 (the reference's request-packed MTP decode through LayerOffload.attend): the union rows
    staged from both tiers, each token's softmax over its own rows; vs the fp64 oracle per token, and vs the
    per-token path (ql = 1) of the same layer."""
    R, ql, nreq, H, K = 4000, 4, 3, 64, 512
    T = ql * nreq
    lo, pool = _offload_layer(dev, R, C, 6, packed=True)
    if C:
        lo.set_hot_rows(torch.arange(0, 2 * C, 2, dtype=torch.int64, device=dev))
    q = make_q(T, H, seed=7)
    g = torch.Generator().manual_seed(8)
    idx = torch.empty(T, K, dtype=torch.int32)
    for r in range(nreq):                          # the tokens of a request share most of their rows
        base = torch.randperm(R, generator=g)[: K + 64]
        for j in range(ql):
            idx[r * ql + j] = base[torch.randperm(K + 64, generator=g)[:K]].to(torch.int32)
    idx[1, 200:] = -1                              # a short row
    idx[5, :] = torch.arange(0, 2 * K, 2)          # all hits when cached
    print(f"[offload packed] C={C} ql={ql} T={T}", flush=True)
    o, lse = lo.attend(q.to(dev), idx.to(dev), SM, 1.0, H, ql=ql, return_lse=True)
    o1, l1 = lo.attend(q.to(dev), idx.to(dev), SM, 1.0, H, ql=1, return_lse=True)
    torch.cuda.synchronize()
    eo, el = ref.attention(q.float().numpy(), pool, idx.numpy(), SM)
    e_o, e_l = _attn_err(o.float().cpu().numpy(), lse.cpu().numpy(), eo, el)
    print(f"[offload packed] err o {e_o:.2e} lse {e_l:.2e}", flush=True)
    assert e_o <= 0 and e_l <= 1e-3
    d_o, d_l = _gpu_diff(o.float().cpu().numpy(), lse.cpu().numpy(), o1.float().cpu().numpy(), l1.cpu().numpy())
    assert d_o <= 1e-2 and d_l <= 1e-4


def _paged_setup(dev, nreq, bs, nb, ctx_len, seed):
    """A paged Row656 cache written through do_kv_cache_update at random slots, plus per-request block tables."""
    from arcagi2_flashnext_dots3_amd.dsa import PortableSparseImpl
    g = torch.Generator().manual_seed(seed)
    nbp = (ctx_len + bs - 1) // bs
    bt = torch.randperm(nb, generator=g)[: nreq * nbp].reshape(nreq, nbp).to(torch.int32)
    pos = torch.arange(ctx_len)
    slots = torch.cat([bt[r, pos // bs].long() * bs + pos % bs for r in range(nreq)])
    n = slots.numel()
    kv = torch.randn(n, 512, generator=g).to(torch.bfloat16)
    pe = torch.randn(n, 1, 64, generator=g).to(torch.bfloat16)
    return PortableSparseImpl, bt, slots, kv, pe


def test_portable_impl_paged_decode(dev):
    from arcagi2_flashnext_dots3_amd.dsa import (CommonAttentionMetadata, PortableSparseBackend)
    nreq, bs, nb, L, H, K = 3, 64, 64, 1000, 128, 256
    Impl, bt, slots, kv, pe = _paged_setup(dev, nreq, bs, nb, L, 6)
    assert PortableSparseBackend.get_impl_cls() is Impl
    cache = torch.zeros(nb, bs, 656, dtype=torch.uint8, device=dev)
    g = torch.Generator().manual_seed(7)
    topk = torch.stack([torch.randperm(L, generator=g)[:K] for _ in range(nreq)]).to(torch.int32)
    topk[1, 200:] = -1
    impl = Impl(H, 576, SM, 1, None, None, "fp8_ds_mla", None, "decoder", None,
                topk_indices_buffer=topk.to(dev), kv_lora_rank=512)
    impl.do_kv_cache_update(kv.to(dev), pe.to(dev), cache, slots.to(dev), "fp8_ds_mla", 1.0)
    builder = PortableSparseBackend.get_builder_cls()(bs, K, 16, dev)
    cam = CommonAttentionMetadata(query_start_loc=torch.arange(nreq + 1, dtype=torch.int32, device=dev),
                                  num_reqs=nreq, num_actual_tokens=nreq, max_query_len=1, max_seq_len=L,
                                  slot_mapping=slots[:nreq].to(dev), block_table_tensor=bt.to(dev))
    md = builder.build(0, cam)
    q = make_q(nreq, H, seed=8)
    out, none = impl.forward_mqa(q.to(dev), cache, md, None)
    torch.cuda.synchronize()
    assert none is None and out.shape == (nreq, H, 512)
    flat = np.zeros((nb * bs, 656), dtype=np.uint8)
    ref.cache_write_656(bf16_bits(kv), bf16_bits(pe.reshape(-1, 64)), slots.numpy(), flat)
    assert np.array_equal(cache.cpu().numpy().reshape(-1, 656), flat)
    rows = ref.rows_from_topk(topk.numpy(), np.arange(nreq), bt.numpy(), bs)
    eo, el = ref.attention(q.float().numpy(), flat, rows, SM)
    assert attn_excess(out.float().cpu().numpy(), eo) <= 0


def test_portable_impl_offload_verify(dev):
    """verify=True (ARC_OFFLOAD_VERIFY): both caches are written, the offload output is checked against the paged
    one on every step and the paged one is returned; on agreeing paths no token is reported."""
    from arcagi2_flashnext_dots3_amd.dsa import (CommonAttentionMetadata, DecodeMetadata, IndexerMetadata,
                                                 PortableSparseBackend)
    nreq, bs, nb, L, H, K = 3, 64, 64, 1000, 64, 256
    Impl, bt, slots, kv, pe = _paged_setup(dev, nreq, bs, nb, L, 16)
    cache = torch.zeros(nb, bs, 656, dtype=torch.uint8, device=dev)
    g = torch.Generator().manual_seed(17)
    topk = torch.stack([torch.randperm(L, generator=g)[:K] for _ in range(nreq)]).to(torch.int32)
    impl = Impl(H, 576, SM, 1, None, None, "fp8_ds_mla", None, "decoder", None, topk_indices_buffer=topk.to(dev),
                offload=True, cache_rows=500, verify=True)
    impl.do_kv_cache_update(kv.to(dev), pe.to(dev), cache, slots.to(dev), "fp8_ds_mla", 1.0)
    impl._off.set_hot_rows(slots[::2][:500].to(dev))
    builder = PortableSparseBackend.get_builder_cls()(bs, K, 16, dev)
    cam = CommonAttentionMetadata(query_start_loc=torch.arange(nreq + 1, dtype=torch.int32, device=dev),
                                  num_reqs=nreq, num_actual_tokens=nreq, max_query_len=1, max_seq_len=L,
                                  slot_mapping=slots[:nreq].to(dev), block_table_tensor=bt.to(dev))
    md = builder.build(0, cam)
    md.indexer = IndexerMetadata(num_decode_tokens=nreq, num_decodes=nreq, num_prefill_tokens=0,
                                 decode=DecodeMetadata(block_table=bt.to(dev), seq_lens=torch.full((nreq,), L, device=dev),
                                                       decode_lens=torch.ones(nreq, device=dev)))
    q = make_q(nreq, H, seed=18)
    print("[offload verify]", flush=True)
    out, _ = impl.forward_mqa(q.to(dev), cache, md, None)
    torch.cuda.synchronize()
    st = impl.verify_stats
    print(f"[offload verify] {st}", flush=True)
    assert st["calls"] == 1 and st["tokens"] == nreq and st["bad"] == 0 and st["max_rel"] < 2e-2
    flat = np.zeros((nb * bs, 656), dtype=np.uint8)
    ref.cache_write_656(bf16_bits(kv), bf16_bits(pe.reshape(-1, 64)), slots.numpy(), flat)
    assert np.array_equal(cache.cpu().numpy().reshape(-1, 656), flat)      # the paged cache was written too
    rows = ref.rows_from_topk(topk.numpy(), np.arange(nreq), bt.numpy(), bs)
    eo, el = ref.attention(q.float().numpy(), flat, rows, SM)
    assert attn_excess(out.float().cpu().numpy(), eo) <= 0


def test_offload_attend_timer(dev):
    """time_every (ARC_OFFLOAD_ATTN2_TIME): every attend call is bracketed by GPU events, read back later without
    a synchronization in the loop; the arm of each call is recorded."""
    R, C, T, H, K = 3000, 800, 4, 64, 256
    lines = []
    lo, _ = _offload_layer(dev, R, C, 19, time_every=3)
    lo.timer.log = lines.append
    lo.set_hot_rows(torch.arange(0, 2 * C, 2, dtype=torch.int64, device=dev))
    q = make_q(T, H, seed=20).to(dev)
    idx = distinct_idx(T, K, R, seed=21).to(dev)
    print("[offload timer]", flush=True)
    for _ in range(5):
        lo.attend(q, idx, SM, 1.0, H)
    assert len(lo.timer.queue) == 5                # nothing read back yet (no wait in the loop)
    stats = lo.timer.drain()
    assert stats["tiers"][0] == 5 and stats["tiers"][1] > 0 and stats["tiers"][2] == 5 * T
    assert lines and lines[0].startswith("[attn time] tiers: n=5")


def test_offload_access_trace(dev, tmp_path):
    """trace= (ARC_OFFLOAD_DUMP): the layer's stores and attend rows go to the npz as the reference's _record lays
    them out; the attention output is the untraced layer's."""
    from arcagi2_flashnext_dots3_amd.diagnostics import AccessTrace
    R, C, T, H, K = 3000, 800, 4, 64, 256
    tr = AccessTrace(tmp_path / "acc", calls=2, unique=True, log=lambda m: None)
    lo, _ = _offload_layer(dev, R, C, 22, trace=tr)          # the store before the first attend is not recorded
    ref_lo, _ = _offload_layer(dev, R, C, 22)
    q = make_q(T, H, seed=23).to(dev)
    idx = distinct_idx(T, K, R, seed=24)
    idx[0, 10:] = -1
    print("[offload trace]", flush=True)
    o = lo.attend(q, idx.to(dev), SM, 1.0, H, slots=torch.arange(5, 9, device=dev))
    assert torch.equal(o, ref_lo.attend(q, idx.to(dev), SM, 1.0, H))
    kv = torch.randn(2, 512).to(torch.bfloat16).to(dev)
    pe = torch.randn(2, 64).to(torch.bfloat16).to(dev)
    lo.store(kv, pe, torch.tensor([40, 41], device=dev))
    lo.attend(q, idx.to(dev), SM, 1.0, H)
    torch.cuda.synchronize()
    z = np.load(tmp_path / "acc.npz")
    want = np.unique(idx.numpy()[idx.numpy() >= 0]).astype(np.int32)
    assert z["kinds"].tolist() == [0, 1, 0, 1] and int(z["C"]) == C and int(z["W"]) == 1 and int(z["R"]) == R
    assert z["e0"].tolist() == [5, 6, 7, 8] and np.array_equal(z["e1"], want)
    assert z["e2"].tolist() == [40, 41] and np.array_equal(z["e3"], want)


def test_offload_hit_rate_stats(dev):
    """stats_every (ARC_OFFLOAD_STATS): every N attend calls one line with the valid rows, the distinct rows and the
    cache's hit rate over them as the call finds it."""
    R, C, T, H, K = 3000, 800, 2, 64, 256
    lines = []
    lo, _ = _offload_layer(dev, R, C, 25, stats_every=2, log=lines.append)
    lo.set_hot_rows(torch.arange(0, 2 * C, 2, dtype=torch.int64, device=dev))     # even rows below 1600
    q = make_q(T, H, seed=26).to(dev)
    idx = torch.full((T, K), -1, dtype=torch.int32)
    idx[0, :100] = torch.arange(0, 200, 2)                  # 100 hits
    idx[1, :100] = torch.arange(1, 200, 2)                  # 100 misses
    idx[1, 100:150] = torch.arange(0, 100, 2)               # 50 hits, repeated from row 0
    print("[offload stats]", flush=True)
    for _ in range(3):
        lo.attend(q, idx.to(dev), SM, 1.0, H)
    torch.cuda.synchronize()
    assert lines == ["[offstats] C=800 rows=250 uniq=200 hit=0.600"]


def test_offload_ways_call_stats(dev):
    """lstats_every (ARC_OFFLOAD_LSTATS): the W-way cache's counts of the call (hits, distinct misses, spill rows)
    with the layer id of the key: a first call misses every distinct valid row, a repeat of it hits every entry."""
    from arcagi2_flashnext_dots3_amd.sparse_offload import LayerOffload
    R, C, T, H, K = 3000, 1024, 2, 64, 256
    lines = []
    lo = LayerOffload(R, dev, key="model.layers.7.self_attn.indexer.k_cache", cache_rows=C, cache_mode="ways",
                      ways=16, lstats_every=1, log=lines.append)
    g = torch.Generator().manual_seed(27)
    lo.store(torch.randn(R, 512, generator=g).to(torch.bfloat16).to(dev),
             torch.randn(R, 64, generator=g).to(torch.bfloat16).to(dev), torch.arange(R, device=dev))
    q = make_q(T, H, seed=28).to(dev)
    idx = distinct_idx(T, K, 400, seed=29)                  # rows below 400: the two tokens share rows
    idx[1, 200:] = -1
    nvalid = int((idx >= 0).sum())
    ndist = int(np.unique(idx.numpy()[idx.numpy() >= 0]).size)
    print("[offload lstats]", flush=True)
    lo.attend(q, idx.to(dev), SM, 1.0, H)
    lo.attend(q, idx.to(dev), SM, 1.0, H)
    torch.cuda.synchronize()
    assert lines[0] == f"[offl] L7 C={C} T={T} n={T * K} hit=0 miss={ndist} spill=0"
    assert lines[1] == f"[offl] L7 C={C} T={T} n={T * K} hit={nvalid} miss=0 spill=0"


def test_portable_impl_offload_decode_and_prefill(dev):
    """Offload mode: decode tokens via LayerOffload.attend, one prefill chunk via staged (compacted) rows; both
    against the oracle over the same rows."""
    from arcagi2_flashnext_dots3_amd.dsa import (DecodeMetadata, IndexerMetadata, PrefillChunk, PrefillMetadata)
    nreq, bs, nb, L, H, K = 2, 64, 40, 900, 64, 128
    Impl, bt, slots, kv, pe = _paged_setup(dev, nreq, bs, nb, L, 10)
    cache = torch.zeros(nb, bs, 656, dtype=torch.uint8, device=dev)
    g = torch.Generator().manual_seed(11)
    nd, npf = 2, 3                                       # 2 decode tokens (one per request), 3 prefill tokens
    topk = torch.full((nd + npf, K), -1, dtype=torch.int32)
    for t in range(nd):
        topk[t] = torch.randperm(L, generator=g)[:K]
    for t in range(npf):                                 # prefill tokens of request 1 at positions 10, 11, 12
        m = 10 + t + 1
        topk[nd + t, :m] = torch.randperm(m, generator=g)
    impl = Impl(H, 576, SM, 1, None, None, "fp8_ds_mla", None, "decoder", None,
                topk_indices_buffer=topk.to(dev), offload=True, cache_rows=1000)
    impl.do_kv_cache_update(kv.to(dev), pe.to(dev), cache, slots.to(dev), "fp8_ds_mla", 1.0)
    impl._off.set_hot_rows(slots[::3][:1000].to(dev))
    # prefill chunk: the context of request 1 is its first 13 positions; rows = that request's slots
    tot = 13
    chunk = PrefillChunk(token_start=nd, token_end=nd + npf, total_seq_lens=tot,
                         token_to_seq=torch.zeros(tot, dtype=torch.int32, device=dev),
                         cu_seq_lens=torch.tensor([0, tot], dtype=torch.int32, device=dev),
                         block_table=bt[1:2].to(dev),
                         cu_seqlen_ks=torch.zeros(npf, dtype=torch.int32, device=dev),
                         cu_seqlen_ke=torch.full((npf,), tot, dtype=torch.int32, device=dev))
    im = IndexerMetadata(num_decode_tokens=nd, num_decodes=nd, num_prefill_tokens=npf,
                         decode=DecodeMetadata(block_table=bt.to(dev), seq_lens=torch.full((nd,), L, device=dev),
                                               decode_lens=torch.ones(nd, device=dev)),
                         prefill=PrefillMetadata(chunks=[chunk]))
    q = make_q(nd + npf, H, seed=12)
    out, _ = impl.forward_mqa(q.to(dev), cache, im, None)
    torch.cuda.synchronize()
    flat = np.zeros((nb * bs, 656), dtype=np.uint8)
    ref.cache_write_656(bf16_bits(kv), bf16_bits(pe.reshape(-1, 64)), slots.numpy(), flat)
    assert np.array_equal(impl._off.host.numpy(), flat)
    rows = np.full((nd + npf, K), -1, dtype=np.int64)
    rows[:nd] = ref.rows_from_topk(topk[:nd].numpy(), np.arange(nd), bt.numpy(), bs)
    rows[nd:] = ref.rows_from_topk(topk[nd:].numpy(), np.ones(npf, dtype=np.int64), bt.numpy(), bs)
    eo, el = ref.attention(q.float().numpy(), flat, rows.astype(np.int32), SM)
    e_o = attn_excess(out.float().cpu().numpy(), eo)
    print(f"[offload impl] excess over the output bar {e_o:.2e}", flush=True)
    assert e_o <= 0


def test_portable_impl_paged_decode_row576(dev):
    """The reference's deployed cache: 576-byte per-tensor fp8 rows ("fp8", dsa_sm89.py:551-562) written with a
    k_scale and attended in place with the layer's _k_scale_float (dsa_sm89.py:379-391), against the fp64 oracle over
    the same Row576 rows; the Row576 -> Row656 gather (kernels.row576_gather) byte-checked too (codes as stored,
    scales 1.0, rope widened: torch's float8_e4m3fn -> bfloat16 conversion)."""
    from types import SimpleNamespace
    from arcagi2_flashnext_dots3_amd import kernels
    from arcagi2_flashnext_dots3_amd.dsa import CommonAttentionMetadata, PortableSparseBackend
    nreq, bs, nb, L, H, K, ks = 3, 64, 64, 1000, 128, 256, 0.05
    Impl, bt, slots, kv, pe = _paged_setup(dev, nreq, bs, nb, L, 16)
    cache = torch.zeros(nb, bs, 576, dtype=torch.uint8, device=dev)
    g = torch.Generator().manual_seed(17)
    topk = torch.stack([torch.randperm(L, generator=g)[:K] for _ in range(nreq)]).to(torch.int32)
    topk[2, 50:] = -1
    impl = Impl(H, 576, SM, 1, None, None, "fp8", None, "decoder", None, topk_indices_buffer=topk.to(dev))
    impl.do_kv_cache_update(kv.to(dev), pe.to(dev), cache, slots.to(dev), "fp8", ks)
    builder = PortableSparseBackend.get_builder_cls()(bs, K, 16, dev)
    cam = CommonAttentionMetadata(query_start_loc=torch.arange(nreq + 1, dtype=torch.int32, device=dev),
                                  num_reqs=nreq, num_actual_tokens=nreq, max_query_len=1, max_seq_len=L,
                                  slot_mapping=slots[:nreq].to(dev), block_table_tensor=bt.to(dev))
    md = builder.build(0, cam)
    q = make_q(nreq, H, seed=18)
    print("[row576] paged decode through PortableSparseImpl", flush=True)
    out, _ = impl.forward_mqa(q.to(dev), cache, md, SimpleNamespace(_k_scale_float=ks))
    torch.cuda.synchronize()
    flat = cache.cpu().numpy().reshape(-1, 576)
    rows = ref.rows_from_topk(topk.numpy(), np.arange(nreq), bt.numpy(), bs)
    eo, el = ref.attention(q.float().numpy(), flat, rows, SM, ks, fmt=576)
    o = out.float().cpu().numpy()
    assert np.all(np.abs(o - eo) <= 1e-2 + 2.0 ** -7 * np.abs(eo).max(axis=-1, keepdims=True))
    # the staging rows themselves
    want = torch.tensor([5, -1, 17, nb * bs, 63, 0], dtype=torch.int64)
    staged = torch.full((6, 656), 0xAB, dtype=torch.uint8, device=dev)
    kernels.row576_gather(cache.view(-1, 576), want.to(dev), staged)
    s = staged.cpu().numpy()
    for i, r in enumerate(want.tolist()):
        if 0 <= r < nb * bs:
            src = flat[r]
            assert np.array_equal(s[i, :512], src[:512])
            assert np.array_equal(s[i, 512:528].view(np.float32), np.ones(4, np.float32))
            rope = torch.from_numpy(src[512:].copy()).view(torch.float8_e4m3fn).to(torch.bfloat16)
            assert np.array_equal(s[i, 528:].view(np.uint16), rope.view(torch.int16).numpy().view(np.uint16))
        else:
            assert not s[i].any()


def test_offload_decode_q_with_extra_heads(dev):
    """q carries more heads than the layer owns (the padded-head layout): the offload path returns the layer's heads
    of LayerOffload.attend's result, equal to the oracle over those heads."""
    from arcagi2_flashnext_dots3_amd.dsa import DecodeMetadata, IndexerMetadata
    nreq, bs, nb, L, Hq, H, K = 2, 64, 40, 900, 128, 64, 128
    Impl, bt, slots, kv, pe = _paged_setup(dev, nreq, bs, nb, L, 20)
    cache = torch.zeros(nb, bs, 656, dtype=torch.uint8, device=dev)
    g = torch.Generator().manual_seed(21)
    topk = torch.stack([torch.randperm(L, generator=g)[:K] for _ in range(nreq)]).to(torch.int32)
    impl = Impl(H, 576, SM, 1, None, None, "fp8_ds_mla", None, "decoder", None, topk_indices_buffer=topk.to(dev),
                offload=True)
    impl.do_kv_cache_update(kv.to(dev), pe.to(dev), cache, slots.to(dev), "fp8_ds_mla", 1.0)
    im = IndexerMetadata(num_decode_tokens=nreq, num_decodes=nreq, num_prefill_tokens=0,
                         decode=DecodeMetadata(block_table=bt.to(dev), seq_lens=torch.full((nreq,), L, device=dev),
                                               decode_lens=torch.ones(nreq, device=dev)))
    q = make_q(nreq, Hq, seed=22)
    print("[offload] q with 128 heads, layer with 64", flush=True)
    out, _ = impl.forward_mqa(q.to(dev), cache, im, None)
    torch.cuda.synchronize()
    assert out.shape == (nreq, H, 512)
    flat = np.zeros((nb * bs, 656), dtype=np.uint8)
    ref.cache_write_656(bf16_bits(kv), bf16_bits(pe.reshape(-1, 64)), slots.numpy(), flat)
    rows = ref.rows_from_topk(topk.numpy(), np.arange(nreq), bt.numpy(), bs)
    eo, _ = ref.attention(q[:, :H].float().numpy(), flat, rows.astype(np.int32), SM)
    assert attn_excess(out.float().cpu().numpy(), eo) <= 0
