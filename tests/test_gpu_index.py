"""GPU parity of the indexer logits (tolerance vs the fp64 oracle, identical -inf pattern) and of the exact top-k
(bit-exact indices vs the oracle on the same fp32 logits, lower index wins ties)."""
import json
import os

import numpy as np
import pytest
import torch

from oracle import spmla_ref as ref
from tests.helpers import bf16_bits

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def _keys(nb, bs, seed):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(nb * bs, 128, generator=g).to(torch.bfloat16)
    store = np.zeros((nb * bs, 132), dtype=np.uint8)
    ref.index_key_write(bf16_bits(k), np.arange(nb * bs), store)
    return store


@pytest.mark.parametrize("rows,L,seed", [(4, 2048, 0), (8, 5000, 1)])
def test_index_logits(dev, rows, L, seed):
    from arcagi2_flashnext_dots3_amd import kernels
    bs = 64
    nbp = (L + bs - 1) // bs
    nb = rows * nbp + 3
    store = _keys(nb, bs, seed + 10)
    g = torch.Generator().manual_seed(seed)
    bt = torch.randperm(nb, generator=g)[: rows * nbp].reshape(rows, nbp).to(torch.int32)
    q = torch.randn(rows, 64, 128, generator=g).to(torch.bfloat16)
    w = torch.rand(rows, 64, generator=g)
    req = torch.arange(rows, dtype=torch.int32)
    ctx = torch.randint(L // 2, L + 1, (rows,), generator=g).to(torch.int32)
    ctx[0] = L
    print(f"[logits] rows={rows} L={L}", flush=True)
    out = kernels.index_logits(q.to(dev), w.to(dev), torch.from_numpy(store).to(dev).view(nb, bs, 132),
                               bt.to(dev), bs, req.to(dev), ctx.to(dev), L)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    exp = ref.index_logits(q.float().numpy(), w.numpy(), store, bt.numpy(), bs, req.numpy(), ctx.numpy(), L)
    assert np.array_equal(np.isinf(got), np.isinf(exp))
    fin = np.isfinite(exp)
    # bound: fp32 accumulation of 128-term dot products and of the 64-head weighted sum (bf16 MFMA, exact products)
    err = np.abs(got[fin] - exp[fin]) / np.maximum(1.0, np.abs(exp[fin]))
    print(f"[logits] max rel err {err.max():.3e}", flush=True)
    assert err.max() <= 2e-5


def _topk_check(dev, lg, ctx, K):
    """The top-k paths against the oracle: several workgroups per row with the full workspace (a narrowing level
    hands its bin's keys to the next in the overflow lists), the same with a workspace too small for those lists (the
    next level reads the row again), and one workgroup per row."""
    from arcagi2_flashnext_dots3_amd import _lib, kernels
    exp = ref.topk(lg, ctx, K)
    nb = int(_lib.lib().spmla_topk_ws_bytes(lg.shape[0], lg.shape[1], K))
    small = torch.empty(nb - 16, dtype=torch.uint8, device=dev)
    for single, ws in ((False, None), (False, small), (True, None)):
        out = kernels.topk(torch.from_numpy(lg).to(dev), torch.from_numpy(ctx).to(dev), K, single_pass=single, ws=ws)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        bad = np.where((got != exp).any(1))[0]
        assert bad.size == 0, f"single_pass={single} ws={'small' if ws is not None else 'full'}: rows {bad[:8]} differ"


def test_index_logits_short_contexts(dev):
    """Ranges shorter than a workgroup's waves (8 rows of 6000 columns: 32 workgroups per row of 6 tiles each for 8
    waves) and rows whose valid keys end inside or before a range (ctx 0, 1, 31, 33, 100, 1500, 1537, 6000): every
    tile below ctx is computed once and columns past ctx are -inf, against the fp64 oracle."""
    from arcagi2_flashnext_dots3_amd import kernels
    rows, L, bs = 8, 6000, 64
    nbp = (L + bs - 1) // bs
    nb = rows * nbp + 2
    store = _keys(nb, bs, 50)
    g = torch.Generator().manual_seed(51)
    bt = torch.randperm(nb, generator=g)[: rows * nbp].reshape(rows, nbp).to(torch.int32)
    q = torch.randn(rows, 64, 128, generator=g).to(torch.bfloat16)
    w = torch.rand(rows, 64, generator=g)
    req = torch.arange(rows, dtype=torch.int32)
    ctx = torch.tensor([0, 1, 31, 33, 100, 1500, 1537, L], dtype=torch.int32)
    print("[logits] short contexts", flush=True)
    out = kernels.index_logits(q.to(dev), w.to(dev), torch.from_numpy(store).to(dev).view(nb, bs, 132),
                               bt.to(dev), bs, req.to(dev), ctx.to(dev), L)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    exp = ref.index_logits(q.float().numpy(), w.numpy(), store, bt.numpy(), bs, req.numpy(), ctx.numpy(), L)
    assert np.array_equal(np.isinf(got), np.isinf(exp))
    fin = np.isfinite(exp)
    err = np.abs(got[fin] - exp[fin]) / np.maximum(1.0, np.abs(exp[fin]))
    assert err.max() <= 2e-5


@pytest.mark.parametrize("dtype,noinf", [(torch.float32, False), (torch.float16, True)])
def test_index_logits_long_workgroup_ranges(dev, dtype, noinf):
    """256 rows of 33,000 columns: with one workgroup per row (as many rows as CUs) a workgroup's range passes the
    32,768 columns it can stage in LDS, so its logits are stored tile by tile; the same rows computed in a 4-row launch
    (ranges staged and written at the end) give the same values bit for bit, row 0 matches the fp64 oracle, and
    columns past ctx are -inf (noinf=False) or left as they were (noinf=True)."""
    from arcagi2_flashnext_dots3_amd import kernels
    rows, L, bs = 256, 33000, 64
    nbp = (L + bs - 1) // bs
    store = _keys(nbp + 1, bs, 40)
    g = torch.Generator().manual_seed(41)
    bt = torch.randperm(nbp + 1, generator=g)[:nbp].view(1, nbp).to(torch.int32)
    q = torch.randn(rows, 64, 128, generator=g).to(torch.bfloat16)
    w = torch.rand(rows, 64, generator=g)
    req = torch.zeros(rows, dtype=torch.int32)                          # every row reads the one key sequence
    ctx = torch.randint(L - 3000, L + 1, (rows,), generator=g).to(torch.int32)
    ctx[0] = L
    st = torch.from_numpy(store).to(dev).view(nbp + 1, bs, 132)
    big = torch.full((rows, L), 7.0, dtype=dtype, device=dev)
    small = torch.full((4, L), 7.0, dtype=dtype, device=dev)
    print(f"[logits] long ranges dtype={dtype} noinf={noinf}", flush=True)
    kernels.index_logits(q.to(dev), w.to(dev), st, bt.to(dev), bs, req.to(dev), ctx.to(dev), L, out=big,
                         noinf=noinf, dtype=dtype)
    kernels.index_logits(q[:4].to(dev), w[:4].to(dev), st, bt.to(dev), bs, req[:4].to(dev), ctx[:4].to(dev), L,
                         out=small, noinf=noinf, dtype=dtype)
    torch.cuda.synchronize()
    assert torch.equal(big[:4].view(torch.int16 if dtype == torch.float16 else torch.int32),
                       small.view(torch.int16 if dtype == torch.float16 else torch.int32))
    got = big.float().cpu().numpy()
    c = ctx.numpy()
    for r in (1, 100, 255):
        tail = got[r, c[r]:]
        assert np.all(tail == 7.0) if noinf else np.all(np.isneginf(tail))
    exp = ref.index_logits(q[:1].float().numpy(), w[:1].numpy(), store, bt.numpy(), bs, req[:1].numpy(),
                           ctx[:1].numpy(), L)
    tol = 2e-5 if dtype == torch.float32 else 2.0 ** -10
    err = np.abs(got[0] - exp[0]) / np.maximum(1.0, np.abs(exp[0]))
    print(f"[logits] long ranges: row 0 max rel err {err.max():.3e}", flush=True)
    assert err.max() <= tol


def test_topk_random_and_lengths(dev):
    g = np.random.default_rng(0)
    rows, L = 16, 32768
    lg = g.standard_normal((rows, L)).astype(np.float32)
    ctx = g.integers(1, L + 1, rows).astype(np.int32)
    ctx[0], ctx[1], ctx[2], ctx[3], ctx[4] = L, 0, 1, 2048, 2049
    print("[topk] random", flush=True)
    _topk_check(dev, lg, ctx, 2048)


def test_topk_ties_and_specials(dev):
    g = np.random.default_rng(1)
    rows, L = 12, 9000
    base = g.standard_normal((rows, L)).astype(np.float32)
    lg = base.copy()
    lg[0] = np.round(base[0] * 8) / 8                                  # ties quantized to 1/8
    lg[1] = np.floor(np.abs(base[1]) * 3).clip(max=4)                  # 5 levels
    lg[2] = np.where(base[2] > 0, 0.0, -0.0).astype(np.float32)        # signed zeros only
    lg[3] = 1.0                                                        # all equal
    lg[4, 100:900] = -np.inf                                           # -inf holes
    lg[5, :] = -np.inf
    lg[5, :10] = 3.0                                                   # fewer finite values than K
    lg[6, 7] = np.nan                                                  # NaN is the largest
    lg[7] = np.round(base[7] * 2) / 2
    lg[8, ::3] = 60000.0                                               # clamped maxima
    ctx = np.full(rows, L, dtype=np.int32)
    ctx[9] = 2047
    ctx[10] = 4000
    print("[topk] ties", flush=True)
    _topk_check(dev, lg, ctx, 2048)


def test_topk_concentrated_values(dev):
    """Logits like the indexer's (mean 280, sd 56): the first 11-bit digit bin of the 2048th value holds more than
    4096 keys, so the workspace path narrows a second level across workgroups; one row of few distinct values falls
    back to the one-workgroup selection; L = 40000 leaves a short last chunk."""
    g = np.random.default_rng(5)
    rows, L = 8, 40000
    lg = (280.0 + 56.0 * g.standard_normal((rows, L))).astype(np.float32)
    lg[1] = np.round(lg[1] / 64) * 64                                   # a handful of distinct values
    ctx = np.full(rows, L, dtype=np.int32)
    ctx[2] = 33000
    print("[topk] concentrated", flush=True)
    _topk_check(dev, lg, ctx, 2048)


def test_topk_bins_around_the_candidate_cap(dev):
    """fp32 rows of 32768 columns whose first-digit boundary bin holds 6000 / 8192 / 8193 / 9000 keys (1000 keys
    above it, K = 2048): bins of at most 8192 keys are resolved by the finishing pass from the candidate list (the
    workspace path's cap at this row length), larger ones by a second collect level; every seventh bin value is the
    same, so the final level resolves ties by column."""
    g = np.random.default_rng(11)
    L = 32768
    sizes = [6000, 8192, 8193, 9000]
    lg = np.empty((len(sizes), L), np.float32)
    for r, nb in enumerate(sizes):
        v = g.uniform(0.0, 200.0, L).astype(np.float32)              # below the bin
        v[:1000] = g.uniform(400.0, 500.0, 1000)                     # above it (same exponent, higher digit)
        vals = g.uniform(256.0, 320.0, nb).astype(np.float32)        # one first-digit bin: [256, 320)
        vals[::7] = 300.0
        v[1000:1000 + nb] = vals
        lg[r] = g.permutation(v)
    ctx = np.full(len(sizes), L, dtype=np.int32)
    print("[topk] bins around the candidate cap", flush=True)
    _topk_check(dev, lg, ctx, 2048)


def test_topk_ctx_lengths_fixture(dev):
    # context lengths from the reference's own fixture (runtime_dataset/ctx_lengths.json), clipped to L
    with open(os.path.join(HERE, "golden", "ctx_lengths.json")) as f:
        cl = json.load(f)["ctx"]
    g = np.random.default_rng(2)
    rows, L = 32, 131072
    ctx = np.array([min(c, L) for c in g.choice(cl, rows)], dtype=np.int32)
    lg = g.standard_normal((rows, L)).astype(np.float32)
    print("[topk] fixture ctx", flush=True)
    _topk_check(dev, lg, ctx, 2048)


def test_logits_then_topk_end_to_end(dev):
    """Indices bit-exact against the oracle's top-k of the GPU's own logits; against the fp64 oracle logits, on every
    row, each position whose logit clears the k-th value by more than the logits tolerance is selected and none that
    falls short of it by more is; rows whose gap at the k-th value exceeds the tolerance select exactly the oracle's
    set (at least one such row is required)."""
    from arcagi2_flashnext_dots3_amd import kernels
    rows, L, bs = 4, 8192, 64
    nbp = L // bs
    store = _keys(rows * nbp, bs, 30)
    g = torch.Generator().manual_seed(31)
    bt = torch.arange(rows * nbp, dtype=torch.int32).reshape(rows, nbp)
    q = torch.randn(rows, 64, 128, generator=g).to(torch.bfloat16)
    w = torch.rand(rows, 64, generator=g)
    req = torch.arange(rows, dtype=torch.int32)
    ctx = torch.full((rows,), L, dtype=torch.int32)
    lg = kernels.index_logits(q.to(dev), w.to(dev), torch.from_numpy(store).to(dev).view(-1, bs, 132), bt.to(dev),
                              bs, req.to(dev), ctx.to(dev), L)
    sel = kernels.topk(lg, ctx.to(dev), 2048).cpu().numpy()
    assert np.array_equal(sel, ref.topk(lg.cpu().numpy(), ctx.numpy(), 2048))
    exp = ref.index_logits(q.float().numpy(), w.numpy(), store, bt.numpy(), bs, req.numpy(), ctx.numpy(), L)
    exact = 0
    for r in range(rows):
        srt = np.sort(exp[r])[::-1]
        kth, tol = srt[2047], 4e-5 * max(1.0, abs(srt[2047]))
        s = set(sel[r].tolist())
        must, never = np.nonzero(exp[r] > kth + tol)[0], np.nonzero(exp[r] < kth - tol)[0]
        assert len(must) >= 1900, f"row {r}: only {len(must)} positions clear the k-th value"
        assert set(must.tolist()) <= s and not (set(never.tolist()) & s), f"row {r}: selection off the oracle's order"
        if srt[2047] - srt[2048] > tol:
            assert s == set(np.argsort(-exp[r], kind="stable")[:2048].tolist())
            exact += 1
    print(f"[index] end to end: {exact} of {rows} rows with a clear gap matched the oracle's set", flush=True)
    assert exact >= 1



@pytest.mark.parametrize("dtype,noinf", [(torch.float32, False), (torch.float16, False), (torch.float32, True)])
def test_logits_hist_topk_matches_separate(dev, dtype, noinf):
    """The first-level top-k histogram built in the logits epilogue (spmla_index_logits_hist, then
    spmla_topk_ws_prehist) against the separate calls on the same inputs: identical logits bit for bit and identical
    positions, which are also the oracle's top-k of those logits. Rows with ctx below Lc (a short last chunk, ctx 0,
    ctx <= K), indexer-like concentrated values on some rows, and (noinf False) a block-table entry missing inside
    ctx, whose keys both paths write as -inf."""
    from arcagi2_flashnext_dots3_amd import kernels
    rows, L, bs, K = 10, 40000, 64, 2048
    nbp = (L + bs - 1) // bs
    nb = rows * nbp + 2
    store = _keys(nb, bs, 60)
    g = torch.Generator().manual_seed(61)
    bt = torch.randperm(nb, generator=g)[: rows * nbp].reshape(rows, nbp).to(torch.int32)
    if not noinf:
        bt[3, 5] = -1
    q = torch.randn(rows, 64, 128, generator=g).to(torch.bfloat16)
    q[6:] = (q[6:].float() * 0.05 + 1.0).to(torch.bfloat16)           # concentrated logits (second radix level)
    w = torch.rand(rows, 64, generator=g)
    req = torch.arange(rows, dtype=torch.int32)
    ctx = torch.full((rows,), L, dtype=torch.int32)
    ctx[1], ctx[2], ctx[4], ctx[5] = 0, 2048, 9000, 33000
    st = torch.from_numpy(store).to(dev).view(nb, bs, 132)
    args = (q.to(dev), w.to(dev), st, bt.to(dev), bs, req.to(dev), ctx.to(dev))
    print(f"[logits+topk fused] dtype={dtype} noinf={noinf}", flush=True)
    lg1 = torch.zeros(rows, L, dtype=dtype, device=dev)
    lg2 = torch.zeros(rows, L, dtype=dtype, device=dev)
    kernels.index_logits(*args, L, out=lg1, noinf=noinf)
    tk1 = kernels.topk(lg1, ctx.to(dev), K)
    _, tk2 = kernels.logits_topk(*args, L, K, lg=lg2, noinf=noinf)
    torch.cuda.synchronize()
    iv = torch.int32 if dtype == torch.float32 else torch.int16
    assert torch.equal(lg1.view(iv), lg2.view(iv)), "logits differ between the fused and the separate path"
    assert torch.equal(tk1, tk2), "positions differ between the fused and the separate path"
    exp = ref.topk(lg1.float().cpu().numpy(), ctx.numpy(), K)
    assert np.array_equal(tk2.cpu().numpy(), exp)

# ---- fp16 logits (the reference's ARC_SHARD_F16OUT buffer) and top-k over fp16 keys
def test_index_logits_f16_is_the_rounded_f32(dev):
    """fp16 logits bit for bit equal to the fp32 launch's logits rounded to nearest even (numpy's float32 -> float16),
    -inf where the fp32 launch has -inf; the fp16 values also within half an fp16 ulp (plus the fp32 bound) of the
    fp64 oracle."""
    from arcagi2_flashnext_dots3_amd import kernels
    rows, L, bs = 6, 5000, 64
    nbp = (L + bs - 1) // bs
    nb = rows * nbp + 3
    store = _keys(nb, bs, 40)
    g = torch.Generator().manual_seed(41)
    bt = torch.randperm(nb, generator=g)[: rows * nbp].reshape(rows, nbp).to(torch.int32)
    q = torch.randn(rows, 64, 128, generator=g).to(torch.bfloat16)
    w = torch.rand(rows, 64, generator=g) * 400.0                      # logits up to the 60000 clamp
    req = torch.arange(rows, dtype=torch.int32)
    ctx = torch.randint(L // 2, L + 1, (rows,), generator=g).to(torch.int32)
    ctx[0] = L
    args = (q.to(dev), w.to(dev), torch.from_numpy(store).to(dev).view(nb, bs, 132), bt.to(dev), bs, req.to(dev),
            ctx.to(dev), L)
    print(f"[logits f16] rows={rows} L={L}", flush=True)
    l32 = kernels.index_logits(*args).cpu().numpy()
    l16 = kernels.index_logits(*args, dtype=torch.float16)
    torch.cuda.synchronize()
    assert l16.dtype == torch.float16
    l16 = l16.cpu().numpy()
    assert np.array_equal(l16.view(np.uint16), l32.astype(np.float16).view(np.uint16))
    assert (l32 == 60000.0).any()                                     # the clamp is exercised
    exp = ref.index_logits(q.float().numpy(), w.numpy(), store, bt.numpy(), bs, req.numpy(), ctx.numpy(), L)
    fin = np.isfinite(exp)
    assert np.array_equal(np.isinf(l16), ~fin)
    ulp = np.spacing(np.abs(exp[fin]).astype(np.float16)).astype(np.float64)
    assert (np.abs(l16[fin].astype(np.float64) - exp[fin]) <= 0.5 * ulp + 2e-5 * np.maximum(1.0, np.abs(exp[fin]))).all()


def _topk16_check(dev, lg16, ctx, K):
    """All fp16 top-k entry points (workspace, one workgroup per row, fixed scratch, local payload) against the oracle
    on the same values widened to fp32 (exact: the fp16 order equals the fp32 order of the widened values)."""
    from arcagi2_flashnext_dots3_amd import kernels
    exp = ref.topk(lg16.astype(np.float32), ctx, K)
    d16, dctx = torch.from_numpy(lg16).to(dev), torch.from_numpy(ctx).to(dev)
    for name, fn in (("ws", lambda: kernels.topk(d16, dctx, K)),
                     ("single", lambda: kernels.topk(d16, dctx, K, single_pass=True)),
                     ("scratch", lambda: kernels.topk_scratch(d16, dctx, K))):
        got = fn().cpu().numpy()
        bad = np.where((got != exp).any(1))[0]
        assert bad.size == 0, f"fp16 {name}: rows {bad[:8]} differ"
    pk = kernels.topk_local(d16, dctx, 0, 1, K).cpu().numpy()
    assert np.array_equal(pk.view(np.uint32), ref.topk_local(lg16.astype(np.float32), ctx, 0, 1, K).view(np.uint32))


def test_topk_f16_ties_and_specials(dev):
    """fp16 keys: heavy ties (every value is one of a few thousand fp16 numbers), signed zeros, NaN, +-inf, short
    rows, and indexer-like concentrated values whose boundary bin needs the second level."""
    g = np.random.default_rng(7)
    rows, L = 12, 40000
    lg = (280.0 + 56.0 * g.standard_normal((rows, L))).astype(np.float16)
    lg[1] = g.standard_normal(L).astype(np.float16)
    lg[2] = np.where(g.standard_normal(L) > 0, 0.0, -0.0).astype(np.float16)
    lg[3, 100:30000] = -np.inf
    lg[4, :] = -np.inf
    lg[4, :10] = 3.0
    lg[5, 7] = np.nan
    lg[6, ::5] = np.inf
    lg[7] = np.float16(60000.0)
    ctx = np.full(rows, L, dtype=np.int32)
    ctx[8], ctx[9], ctx[10] = 0, 2047, 2049
    print("[topk f16] ties and specials", flush=True)
    _topk16_check(dev, lg, ctx, 2048)


def test_logits_f16_then_topk(dev):
    """The reference's fp16 mode end to end: fp16 logits of the GPU, then top-k on them, bit-exact vs the oracle's
    top-k of the same fp16 values."""
    from arcagi2_flashnext_dots3_amd import kernels
    rows, L, bs = 4, 8192, 64
    nbp = L // bs
    store = _keys(rows * nbp, bs, 50)
    g = torch.Generator().manual_seed(51)
    bt = torch.arange(rows * nbp, dtype=torch.int32).reshape(rows, nbp)
    q = torch.randn(rows, 64, 128, generator=g).to(torch.bfloat16)
    w = torch.rand(rows, 64, generator=g)
    req = torch.arange(rows, dtype=torch.int32)
    ctx = torch.full((rows,), L, dtype=torch.int32)
    ctx[1] = L - 1000
    print("[logits f16 + topk]", flush=True)
    lg = kernels.index_logits(q.to(dev), w.to(dev), torch.from_numpy(store).to(dev).view(-1, bs, 132), bt.to(dev),
                              bs, req.to(dev), ctx.to(dev), L, dtype=torch.float16)
    sel = kernels.topk(lg, ctx.to(dev), 2048).cpu().numpy()
    assert np.array_equal(sel, ref.topk(lg.cpu().numpy().astype(np.float32), ctx.numpy(), 2048))
