"""GPU parity at the BASELINE configs' full sizes, through the C-ABI, on the same seeded inputs bench.py times: the GPU
runs every token / row of the full launch; the fp64 oracle checks a sample of them (its cost grows with the sample,
not the launch), and what no sample covers is checked by size-independent properties (the single-pass attention vs
the split one on every token, top-k bit-exact on every row of the GPU's own logits). Output bar for these N(0, 1)
workloads: |o - ref| <= 1e-2 + half a bf16 ulp of ref; lse within 1e-3; logits within 2e-5 relative (fp32
accumulation of 128-term dot products and of the 64-head weighted sum)."""
import numpy as np
import pytest
import torch

from oracle import spmla_ref as ref
from tests.helpers import attn_excess

pytestmark = pytest.mark.gpu


def _check_rows(o, l, o_ref, l_ref, what):
    fin = np.isfinite(l_ref)
    assert np.array_equal(fin, np.isfinite(l)), f"{what}: lse -inf pattern"
    viol = attn_excess(o, o_ref)
    assert viol <= 0, f"{what}: output {viol:.3e} beyond the bar"
    if fin.any():
        assert np.abs(l[fin] - l_ref[fin]).max() <= 1e-3, f"{what}: lse"


def _oracle_tokens(q, pool, idx, tokens, sm, kv_scale=1.0):
    """The oracle over the listed tokens: their selected rows copied from the device pool, indices remapped."""
    sel = idx[tokens].to(torch.int64)
    valid = (sel >= 0) & (sel < pool.shape[0])
    rows = pool[sel.clamp(0, pool.shape[0] - 1).reshape(-1)].cpu().numpy()
    local = np.where(valid.cpu().numpy(), np.arange(sel.numel()).reshape(sel.shape), -1)
    return ref.attention(q[tokens].float().cpu().numpy(), rows, local, sm, kv_scale)


def test_config2_full_size(dev):
    """B=64, 128 heads, top-2048 of 32768 rows per sequence over the 2,097,152-row pool (the last
    sequence's rows sit at byte offsets up to 1.38e9); the default launch (the head-group kernel, unsplit) vs the
    oracle on 8 tokens spread over the batch, and vs the 128-head kernel with its in-kernel merge of 4 splits
    on every token."""
    import bench
    from arcagi2_flashnext_dots3_amd import kernels
    pool, q, idxs = bench.build_inputs(dev, 1)
    idx = idxs[0]
    assert pool.shape[0] == 2097152 and int(idx.max()) >= 2097152 - 32768
    print("[fullsize] config 2: B=64, 2M-row pool", flush=True)
    assert kernels.auto_split(64, 128, 2048) == 1
    out, lse = kernels.attend(q, pool, idx, bench.SM_SCALE)
    o1, l1 = kernels.attend(q, pool, idx, bench.SM_SCALE, split=4)
    torch.cuda.synchronize()
    tokens = [0, 9, 18, 27, 36, 45, 54, 63]
    o_ref, l_ref = _oracle_tokens(q, pool, idx, tokens, bench.SM_SCALE)
    _check_rows(out[tokens].float().cpu().numpy(), lse[tokens].cpu().numpy(), o_ref, l_ref, "config 2")
    # both bf16 (at most one rounding step, 2^-7 relative, apart) with f16 P' / partials whose rounding (2^-11 per term)
    # is relative to the head's terms, so it stays of that size where they cancel into a small output value
    o1f = o1.float()
    bar = 2.0 ** -7 * o1f.abs() + 2.0 ** -9 * o1f.abs().amax(dim=-1, keepdim=True) + 1e-5
    assert float(((out.float() - o1f).abs() - bar).max()) <= 0 and float((lse - l1).abs().max()) <= 1e-5


def test_config3_full_size(dev):
    """the 2,097,152-row pool in pinned host memory behind the HBM hot set of its 524,288 most
    frequent rows over the bench's 64 steps of Zipf(1.1) warm-up draws; a step of B=64 Zipf selections through the two tiers (HBM-tier
    attention + host rows over PCIe + merge) vs the oracle over the host rows on 8 tokens spread over the batch."""
    import bench
    from arcagi2_flashnext_dots3_amd.sparse_offload import LayerOffload, hot_rows_by_frequency
    R, C, B, K = bench.R3, bench.R3 // 4, bench.B, bench.K
    lo = LayerOffload(R, dev, cache_rows=C)
    bench._cache_fill(lo.host, R, 1, dev)
    perm = torch.randperm(R, generator=torch.Generator().manual_seed(3))
    warm = bench.zipf_selections(64 * B, K, R, seed=4, perm=perm, device=dev)
    lo.set_hot_rows(hot_rows_by_frequency(torch.bincount(warm.reshape(-1), minlength=R), C))
    del warm
    idx = bench.zipf_selections(B, K, R, seed=5, perm=perm, device=dev).to(torch.int32)
    q = torch.randn(B, bench.H, 576, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16).to(dev)
    hit = lo.hit_rate(idx)
    print(f"[fullsize] config 3: 2M pinned rows, hit rate {hit:.3f}", flush=True)
    assert 0.2 < hit < 1.0                                 # both tiers carry rows
    out, lse = lo.attend(q, idx, bench.SM_SCALE, 1.0, bench.H, return_lse=True)
    torch.cuda.synchronize()
    tokens = [0, 9, 18, 27, 36, 45, 54, 63]
    host = lo.host.numpy()
    sel = idx[tokens].cpu().numpy().astype(np.int64)
    rows = host[sel.reshape(-1)]
    local = np.arange(sel.size).reshape(sel.shape)
    o_ref, l_ref = ref.attention(q[tokens].float().cpu().numpy(), rows, local, bench.SM_SCALE)
    _check_rows(out[tokens].float().cpu().numpy(), lse[tokens].cpu().numpy(), o_ref, l_ref, "config 3")


@pytest.mark.parametrize("L,B", [(32768, 64), (131072, 64)])
def test_config4_full_size(dev, L, B):
    """indexer logits over L keys per sequence (a scattered block table over the key cache) for
    every row of the launch, the fp64 oracle on 3 rows; top-2048 bit-exact against the oracle's selection on the
    GPU's own fp32 logits for every row; the fused step (histogram in the logits epilogue) gives the same logits bit
    for bit and the same positions."""
    from arcagi2_flashnext_dots3_amd import kernels
    from arcagi2_flashnext_dots3_amd.shard_indexer import ShardStore
    bs, K = 64, 2048
    nbp = L // bs
    kc = torch.empty(B * nbp + 5, bs, 132, dtype=torch.uint8, device=dev)
    st = ShardStore(kc, 1, 0)
    g = torch.Generator(device=dev).manual_seed(5)
    for r0 in range(0, kc.shape[0] * bs, 1 << 20):
        n = min(1 << 20, kc.shape[0] * bs - r0)
        st.write(torch.randn(n, 128, generator=g, device=dev).to(torch.bfloat16),
                 torch.arange(r0, r0 + n, dtype=torch.int64, device=dev), False)
    bt = torch.randperm(kc.shape[0], generator=torch.Generator().manual_seed(6))[: B * nbp]
    bt = bt.view(B, nbp).to(torch.int32).to(dev)
    q = torch.randn(B, 64, 128, generator=torch.Generator().manual_seed(7)).to(torch.bfloat16).to(dev)
    w = torch.rand(B, 64, generator=torch.Generator().manual_seed(8)).to(dev)
    req = torch.arange(B, dtype=torch.int32, device=dev)
    ctx = torch.full((B,), L, dtype=torch.int32, device=dev)
    ctx[1] = L - 777                                       # a shorter row: -inf beyond its context
    print(f"[fullsize] config 4: L={L}, {B} rows", flush=True)
    lg = kernels.index_logits(q, w, kc, bt, bs, req, ctx, L)
    top = kernels.topk(lg, ctx, K)
    # the step as ShardStore.logits_topk runs it: the top-k's first histogram in the logits epilogue
    lg2, top2 = kernels.logits_topk(q, w, kc, bt, bs, req, ctx, L, K)
    torch.cuda.synchronize()
    assert torch.equal(lg2[:, :L].view(torch.int32), lg.view(torch.int32)), "fused logits differ"
    assert torch.equal(top2, top), "fused positions differ"
    got = lg.cpu().numpy()
    for r in (0, 1, B - 1):                                # oracle on the blocks of three rows
        blocks = bt[r].long()
        store = kc[blocks].reshape(-1, 132).cpu().numpy()
        local_bt = np.arange(nbp, dtype=np.int32).reshape(1, nbp)
        exp = ref.index_logits(q[r:r + 1].float().cpu().numpy(), w[r:r + 1].cpu().numpy(), store, local_bt, bs,
                               np.zeros(1, np.int32), ctx[r:r + 1].cpu().numpy(), L)[0]
        assert np.array_equal(np.isinf(got[r]), np.isinf(exp))
        fin = np.isfinite(exp)
        assert (np.abs(got[r][fin] - exp[fin]) / np.maximum(1.0, np.abs(exp[fin]))).max() <= 2e-5
    assert np.array_equal(top.cpu().numpy(), ref.topk(got, ctx.cpu().numpy(), K))


def test_config5_full_size(dev):
    """one prefill chunk of 8192 queries x 128 heads, each over 2048 selected positions of the
    <= 65536 prior rows of a paged cache (a launch of 8192 workgroups); the oracle on 8 queries spread over the chunk."""
    from arcagi2_flashnext_dots3_amd import kernels
    NQ, CTXMAX, bs, K, H = 8192, 65536, 64, 2048, 128
    nblk = CTXMAX // bs + 64
    cache = torch.zeros(nblk, bs, 656, dtype=torch.uint8, device=dev)
    bt = torch.randperm(nblk, generator=torch.Generator().manual_seed(10))[: CTXMAX // bs]
    bt = bt.to(torch.int32).view(1, -1).to(dev)
    pos = torch.arange(CTXMAX, device=dev)
    slots = bt[0, pos // bs].long() * bs + pos % bs
    g = torch.Generator(device=dev).manual_seed(1)
    for r0 in range(0, CTXMAX, 1 << 16):
        n = min(1 << 16, CTXMAX - r0)
        kernels.cache_write(torch.randn(n, 512, generator=g, device=dev).to(torch.bfloat16),
                            torch.randn(n, 64, generator=g, device=dev).to(torch.bfloat16), slots[r0:r0 + n], cache)
    pos0 = CTXMAX - NQ                                     # query i sees positions [0, pos0 + i]
    vis = torch.arange(pos0 + 1, CTXMAX + 1, device=dev, dtype=torch.float64).view(NQ, 1)
    gp = torch.Generator(device=dev).manual_seed(8)
    tk = (torch.rand(NQ, K, generator=gp, device=dev, dtype=torch.float64) * vis).long().to(torch.int32)
    rows = kernels.rows_from_topk(tk, torch.zeros(NQ, dtype=torch.int32, device=dev), bt, bs)
    q = torch.randn(NQ, H, 576, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16).to(dev)
    flat = cache.view(-1, 656)
    print("[fullsize] config 5: 8192 queries", flush=True)
    out, lse = kernels.attend(q, flat, rows, 192 ** -0.5)
    torch.cuda.synchronize()
    tokens = [0, 1000, 2047, 3333, 4095, 5000, 7000, NQ - 1]
    o_ref, l_ref = _oracle_tokens(q, flat, rows, tokens, 192 ** -0.5)
    _check_rows(out[tokens].float().cpu().numpy(), lse[tokens].cpu().numpy(), o_ref, l_ref, "config 5")
