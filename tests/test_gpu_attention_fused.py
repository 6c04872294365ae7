"""GPU parity of the in-kernel split merge (spmla_attn) and of the f16 range guard of P' = P * scale, against the fp64
oracle through the C-ABI. Output bar: 1e-2 plus one bf16 ulp (2^-7 relative) of the head's largest reference value:
the output's own rounding takes up to half an ulp, and the f16 P' and f16 partials add 2^-11 of the terms they round
-- terms of the head's magnitude, also where they cancel into a small output value. For O(1) outputs this is the 1e-2
bar; at the outputs of ~1e6 that the wide-scale rows give, no absolute bar below it is reachable. lse within 1e-3."""
import numpy as np
import pytest
import torch

from oracle import spmla_ref as ref
from tests.helpers import bf16_bits, distinct_idx, make_pool_656, make_q

pytestmark = pytest.mark.gpu
OUT_TOL, LSE_TOL = 1e-2, 1e-3


def _pool_mag(mags, seed):
    """Row656 rows whose latent is N(0, mags[r]^2) (rope N(0, 1)), packed by the oracle's writer."""
    R = len(mags)
    g = torch.Generator().manual_seed(seed)
    kv = torch.randn(R, 512, generator=g) * torch.as_tensor(mags, dtype=torch.float32)[:, None]
    pe = torch.randn(R, 64, generator=g)
    pool = np.zeros((R, 656), np.uint8)
    ref.cache_write_656(bf16_bits(kv), bf16_bits(pe), np.arange(R), pool)
    return pool


def _run(dev, q, pool, idx, sm, kv=1.0, split=None, kcount=None):
    from arcagi2_flashnext_dots3_amd import kernels
    out, lse = kernels.attend(q.to(dev), torch.from_numpy(pool).to(dev), idx.to(dev), sm, kv, split=split,
                              kcount=None if kcount is None else kcount.to(dev))
    torch.cuda.synchronize()
    return out.float().cpu().numpy(), lse.cpu().numpy()


def _vs_oracle(o, l, o_ref, l_ref):
    fin = np.isfinite(l_ref)
    assert np.array_equal(fin, np.isfinite(l)), "lse -inf pattern differs"
    assert np.all(o[~fin] == 0)
    err = np.abs(o - o_ref) - (OUT_TOL + 2.0 ** -7 * np.abs(o_ref).max(axis=-1, keepdims=True))
    w = np.unravel_index(err.argmax(), err.shape)
    rel = abs(o[w] - o_ref[w]) / max(abs(o_ref[w]), 1e-30)
    assert err.max() <= 0, f"output off by {err.max():.3e} beyond the bar at {w}: {o[w]} vs {o_ref[w]} ({rel:.2e} rel)"
    if fin.any():
        assert np.abs(l[fin] - l_ref[fin]).max() <= LSE_TOL


@pytest.mark.parametrize("split", [2, 3, 4, 5, 8])
def test_fused_split_vs_oracle(dev, split):
    """S splits merged in the kernel: two head groups (the second with 32 heads), ragged per-token counts (splits with
    no rows, a token with none), an invalid tail, kv_scale != 1; equal to the single pass up to the f16 partials, and
    a second launch on the same workspace gives the same bits (the arrival counters reset themselves)."""
    T, H, R, K = 5, 160, 4096, 1536
    pool, _, _ = make_pool_656(R, seed=31)
    q = make_q(T, H, seed=32)
    idx = distinct_idx(T, K, R, seed=33)
    idx[1, 700:] = -1
    kc = torch.tensor([1536, 1000, 0, 333, 1], dtype=torch.int32)
    sm = 192 ** -0.5
    print(f"[fused] T={T} H={H} K={K} split={split}", flush=True)
    o, l = _run(dev, q, pool, idx, sm, 0.7, split=split, kcount=kc)
    o_ref, l_ref = ref.attention(q.float().numpy(), pool, idx.numpy(), sm, 0.7, kcount=kc.numpy())
    _vs_oracle(o, l, o_ref, l_ref)
    o1, l1 = _run(dev, q, pool, idx, sm, 0.7, split=1, kcount=kc)
    # both bf16 (one rounding step, 2^-7 relative, apart) with f16 P' / partials whose rounding (2^-11 per term) is
    # relative to the head's terms, so it stays of that size where they cancel into a small output value
    viol = np.abs(o - o1) - (2.0 ** -7 * np.abs(o1) + 2.0 ** -9 * np.abs(o1).max(axis=-1, keepdims=True) + 1e-5)
    w = np.unravel_index(viol.argmax(), viol.shape)
    assert viol.max() <= 0, f"fused vs single pass at {w}: {o[w]} vs {o1[w]} (oracle {o_ref[w]}), lse {l[w[:2]]} {l1[w[:2]]}"
    fin = np.isfinite(l1)
    assert np.abs(l[fin] - l1[fin]).max() <= 1e-5
    o2, l2 = _run(dev, q, pool, idx, sm, 0.7, split=split, kcount=kc)
    assert np.array_equal(o, o2) and np.array_equal(l, l2)


@pytest.mark.parametrize("case", ["tiny", "huge", "rising", "falling"])
@pytest.mark.parametrize("split", [1, 4])
def test_row_scale_range(dev, case, split):
    """Row scales from 2^-18 to 2^10 (latent magnitudes 1e-3 .. 4e5): P' = P * scale stays in f16's range through the
    power-of-two factor the kernel carries (set by the first tile with a positive scale, raised when a later tile's
    largest scale needs it: "rising" orders the rows by magnitude, so it rises tile after tile)."""
    R, T, H, K = 3072, 2, 128, 1024
    if case == "tiny":
        mags, qs = np.full(R, 1e-3), 1.0
    elif case == "huge":
        mags, qs = np.full(R, 4e5), 1e-3
    else:
        mags, qs = 10.0 ** np.linspace(-3, 5.6, R), 1e-3
    pool = _pool_mag(mags, seed=41)
    q = make_q(T, H, seed=42, scale=qs)
    idx = torch.stack([torch.arange(0, R, 3), torch.arange(1, R, 3)]).to(torch.int32)[:, :K]
    if case == "falling":
        idx = idx.flip(1).contiguous()
    sm = 192 ** -0.5
    print(f"[scale] case={case} split={split}", flush=True)
    o, l = _run(dev, q, pool, idx, sm, split=split)
    o_ref, l_ref = ref.attention(q.float().numpy(), pool, idx.numpy(), sm)
    _vs_oracle(o, l, o_ref, l_ref)
    if case == "tiny":      # outputs ~1e-3: also within 2^-8 of their own scale, not only the absolute bar
        assert np.abs(o - o_ref).max() <= 2.0 ** -8 * np.abs(o_ref).max()


def test_workspace_reuse_larger_counter_region(dev):
    """The cached workspace reused by a launch whose counters take more bytes than the previous launch's (bytes that
    launch used as scratch): attend clears them first, and every token of the second launch is merged."""
    from arcagi2_flashnext_dots3_amd import kernels
    R, H, K = 4096, 128, 256
    pool = torch.from_numpy(make_pool_656(R, seed=51)[0]).to(dev)
    sm = 192 ** -0.5
    print("[fused] workspace reuse: T=100 split 8, then T=399 split 2", flush=True)
    kernels.attend(make_q(100, H, seed=52).to(dev), pool, distinct_idx(100, K, R, seed=53).to(dev), sm, split=8)
    T = 399
    assert kernels.attn_ws_bytes(T, H, 2) <= kernels.attn_ws_bytes(100, H, 8)       # served by the same buffer
    q, idx = make_q(T, H, seed=54).to(dev), distinct_idx(T, K, R, seed=55).to(dev)
    out = torch.full((T, H, 512), float("nan"), dtype=torch.bfloat16, device=dev)
    lse = torch.full((T, H), float("nan"), device=dev)
    kernels.attend(q, pool, idx, sm, split=2, out=out, lse=lse)
    o1, l1 = kernels.attend(q, pool, idx, sm, split=1)
    torch.cuda.synchronize()
    o, o1 = out.float(), o1.float()
    bar = 2.0 ** -7 * o1.abs() + 2.0 ** -9 * o1.abs().amax(dim=-1, keepdim=True) + 1e-5
    assert bool(torch.isfinite(o).all()) and float(((o - o1).abs() - bar).max()) <= 0
    assert float((lse - l1).abs().max()) <= 1e-5


def test_graph_capture_ascending_batches(dev):
    """Two decode batches captured in ascending size without an explicit workspace (the serving path's calls): both
    captures use the workspace reserved by an earlier eager call, so neither frees or swaps the other's buffer. Each
    graph is replayed three times, alternating, with eager launches between the replays; every replay equals the
    eager result bit for bit (same kernel, same split, same fixed merge order)."""
    from arcagi2_flashnext_dots3_amd import kernels
    R, H, K = 4096, 128, 2048
    pool = torch.from_numpy(make_pool_656(R, seed=61)[0]).to(dev)
    sm = 192 ** -0.5
    kernels.reserve_workspace(dev, H)
    Ts = (4, 16)
    assert all(kernels.auto_split(T, H, K) > 1 for T in Ts)
    qs = [make_q(T, H, seed=62 + T).to(dev) for T in Ts]
    ids = [distinct_idx(T, K, R, seed=63 + T).to(dev) for T in Ts]
    print(f"[fused] graph capture of T={Ts} (splits {[kernels.auto_split(T, H, K) for T in Ts]})", flush=True)
    eager = [kernels.attend(q, pool, i, sm) for q, i in zip(qs, ids)]
    torch.cuda.synchronize()
    graphs, outs = [], []
    for q, i in zip(qs, ids):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            kernels.attend(q, pool, i, sm)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            outs.append(kernels.attend(q, pool, i, sm))
        torch.cuda.synchronize()
        graphs.append(g)
    for rep in range(3):
        for n in (0, 1):
            outs[n][0].fill_(7.0)
            outs[n][1].fill_(7.0)
            graphs[n].replay()
            torch.cuda.synchronize()
            assert torch.equal(outs[n][0], eager[n][0]), f"replay {rep} of T={Ts[n]}: output differs from eager"
            assert torch.equal(outs[n][1], eager[n][1]), f"replay {rep} of T={Ts[n]}: lse differs from eager"
            o, l = kernels.attend(qs[1 - n], pool, ids[1 - n], sm)       # eager work between the replays
            torch.cuda.synchronize()
            assert torch.equal(o, eager[1 - n][0]) and torch.equal(l, eager[1 - n][1])


def test_auto_split_large_k_single_token(dev):
    """One token over K = 20000 rows with the default split: auto_split returns 1 (every split of 8 would exceed the
    split kernel's 2048-row limit), so the head-group kernel takes any K; the result matches the fp64 oracle."""
    from arcagi2_flashnext_dots3_amd import kernels
    T, H, R, K = 1, 128, 30000, 20000
    assert kernels.auto_split(T, H, K) == 1
    pool = make_pool_656(R, seed=71)[0]
    q = make_q(T, H, seed=72)
    idx = distinct_idx(T, K, R, seed=73)
    sm = 192 ** -0.5
    print("[fused] T=1 K=20000 default split", flush=True)
    o, l = _run(dev, q, pool, idx, sm)
    o_ref, l_ref = ref.attention(q.float().numpy(), pool, idx.numpy(), sm)
    _vs_oracle(o, l, o_ref, l_ref)


def test_first_launches_from_two_threads(dev):
    """The first attention launches of a fresh process, issued from two host threads at once (the per-device dynamic
    LDS attribute is set under a lock by whichever thread comes first): both results equal a later single-threaded
    launch bit for bit."""
    import os
    import subprocess
    import sys
    code = r"""
import threading, torch, sys
sys.path.insert(0, %r)
from arcagi2_flashnext_dots3_amd import kernels
from tests.helpers import make_pool_656, make_q, distinct_idx
dev = torch.device("cuda:0")
pool = torch.from_numpy(make_pool_656(3000, seed=81)[0]).to(dev)
q = make_q(8, 128, seed=82).to(dev)
idx = distinct_idx(8, 512, 3000, seed=83).to(dev)
res, err = [None, None], []
def go(i):
    try:
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            o, l = kernels.attend(q, pool, idx, 192 ** -0.5, split=1)
        s.synchronize()
        res[i] = (o, l)
    except Exception as e:
        err.append(repr(e))
ts = [threading.Thread(target=go, args=(i,)) for i in range(2)]
[t.start() for t in ts]; [t.join() for t in ts]
assert not err, err
o, l = kernels.attend(q, pool, idx, 192 ** -0.5, split=1)
torch.cuda.synchronize()
for r in res:
    assert torch.equal(r[0], o) and torch.equal(r[1], l)
print("two-thread first launches ok")
""" % os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("[fused] first launches from two threads (child process)", flush=True)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=240)
    assert r.returncode == 0 and "two-thread first launches ok" in r.stdout, (r.stdout[-500:], r.stderr[-1500:])
