"""GPU parity of the Row576 attention (spmla_attn576: the plugin's per-tensor fp8 cache, 512 + 64 e4m3 codes per row
and one kv_scale) against the fp64 oracle through the C-ABI: config 1's and config 2's shapes, ragged / invalid /
kcount entries, head counts that are not a multiple of 32, a per-tensor scale other than 1, splits merged through
fp32 partials, and the plugin's paged path at prefill scale with its memory bounded. Output bar: 1e-2 plus half a
bf16 ulp of the reference value (attn_excess); lse within 1e-3."""
import numpy as np
import pytest
import torch

from oracle import spmla_ref as ref
from tests.helpers import attn_excess, distinct_idx, make_pool_576, make_q

pytestmark = pytest.mark.gpu


def _check(o, l, o_ref, l_ref, what):
    fin = np.isfinite(l_ref)
    assert np.array_equal(fin, np.isfinite(l)), f"{what}: lse -inf pattern differs"
    assert np.all(o[~fin] == 0), f"{what}: tokens without rows must give 0"
    viol = attn_excess(o, o_ref)
    assert viol <= 0, f"{what}: output {viol:.3e} beyond the bar"
    if fin.any():
        assert np.abs(l[fin] - l_ref[fin]).max() <= 1e-3, f"{what}: lse"


def _attend(dev, q, pool, idx, sm, kv=1.0, split=None, kcount=None):
    from arcagi2_flashnext_dots3_amd import kernels
    out, lse = kernels.attend(q.to(dev), torch.from_numpy(pool).to(dev), idx.to(dev), sm, kv, split=split,
                              kcount=None if kcount is None else kcount.to(dev))
    torch.cuda.synchronize()
    return out.float().cpu().numpy(), lse.cpu().numpy()


@pytest.mark.parametrize("T,H,R,K,kv,split", [
    (1, 16, 4096, 256, 1.0, 1),        # config 1's shape
    (1, 16, 4096, 256, 1.0, None),     # the same, auto split (fp32 partials + merge)
    (5, 48, 3000, 700, 0.37, 1),       # ragged K, 48 heads (a partial head group), kv_scale != 1
    (3, 128, 8192, 2048, 2.5, 4),      # 128 heads, 4 splits
    (2, 64, 1000, 33, 1.0, 1),         # one full tile and a 1-row tile
])
def test_attn576_vs_oracle(dev, T, H, R, K, kv, split):
    print(f"[576] T={T} H={H} R={R} K={K} kv={kv} split={split}", flush=True)
    pool = make_pool_576(R, seed=R + K, kv_scale=kv)
    q = make_q(T, H, seed=T + H)
    idx = distinct_idx(T, K, R, seed=K)
    sm = 192 ** -0.5
    o, l = _attend(dev, q, pool, idx, sm, kv, split)
    o_ref, l_ref = ref.attention(q.float().numpy(), pool, idx.numpy(), sm, kv, fmt=576)
    _check(o, l, o_ref, l_ref, "Row576")


def test_attn576_invalid_entries_and_kcount(dev):
    """-1, rows past R and entries past kcount contribute nothing; a token with no valid entry gives o = 0,
    lse = -inf; NaN codes in a row nobody selects never reach the output."""
    T, H, R, K = 4, 32, 2048, 300
    pool = make_pool_576(R, seed=7)
    pool[0, :] = 0x7F                                      # e4m3 NaN codes in row 0, which no token selects
    q = make_q(T, H, seed=8)
    idx = distinct_idx(T, K, R - 1, seed=9) + 1
    idx[0, ::3] = -1
    idx[1, 5::7] = R + 11
    idx[2, :] = -1                                         # no valid entry
    kcount = torch.tensor([K, 200, K, 37], dtype=torch.int32)
    sm = 192 ** -0.5
    for split in (1, 2):
        print(f"[576] invalid entries, split {split}", flush=True)
        o, l = _attend(dev, q, pool, idx, sm, split=split, kcount=kcount)
        o_ref, l_ref = ref.attention(q.float().numpy(), pool, idx.numpy(), sm, kcount=kcount.numpy(), fmt=576)
        assert np.isneginf(l[2]).all() and np.all(o[2] == 0)
        _check(o, l, o_ref, l_ref, f"Row576 invalid entries, split {split}")


def test_attn576_config2_shape(dev):
    """Config 2's decode shape over a Row576 pool (B=64, 128 heads, top-2048 of 32768 rows per sequence): the oracle
    on 8 tokens spread over the batch; split and unsplit launches agree."""
    from arcagi2_flashnext_dots3_amd import kernels
    B, H, CTX, K = 64, 128, 32768, 2048
    R = B * CTX
    g = torch.Generator(device=dev).manual_seed(1)
    pool = torch.empty(R, 576, dtype=torch.uint8, device=dev)
    for r0 in range(0, R, 1 << 20):                         # e4m3 codes of N(0, 1) values (|x| <= 448)
        n = min(1 << 20, R - r0)
        pool[r0:r0 + n] = torch.randn(n, 576, generator=g, device=dev).to(torch.float8_e4m3fn).view(torch.uint8)
    gi = torch.Generator(device=dev).manual_seed(2)
    idx = torch.stack([torch.randperm(CTX, generator=gi, device=dev)[:K] + b * CTX for b in range(B)]).to(torch.int32)
    q = torch.randn(B, H, 576, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16).to(dev)
    sm = 192 ** -0.5
    print("[576] config 2 shape", flush=True)
    out, lse = kernels.attend(q, pool, idx, sm, 1.0, split=1)
    o4, l4 = kernels.attend(q, pool, idx, sm, 1.0, split=4)
    torch.cuda.synchronize()
    tokens = [0, 9, 18, 27, 36, 45, 54, 63]
    sel = idx[tokens].long()
    rows = pool[sel.reshape(-1)].cpu().numpy()
    local = np.arange(sel.numel()).reshape(sel.shape)
    o_ref, l_ref = ref.attention(q[tokens].float().cpu().numpy(), rows, local, sm, fmt=576)
    _check(out[tokens].float().cpu().numpy(), lse[tokens].cpu().numpy(), o_ref, l_ref, "Row576 config 2")
    o4f = o4.float()
    bar = 2.0 ** -7 * o4f.abs() + 2.0 ** -9 * o4f.abs().amax(dim=-1, keepdim=True) + 1e-5
    assert float(((out.float() - o4f).abs() - bar).max()) <= 0 and float((lse - l4).abs().max()) <= 1e-5


def test_plugin_row576_paged_prefill_scale(dev):
    """The plugin's Row576 ("fp8") paged cache attended in place at prefill scale (PortableSparseImpl._run: 2048
    tokens x top-2048 over a 65536-row paged cache whose block stride is padded past its rows): the oracle on 8
    tokens, and no staging copy -- the memory the call adds stays below 0.6 GB (the output and the launch's own
    buffers), where a Row656 copy of the selected rows would take 2048 x 2048 x 656 B = 2.75 GB."""
    from arcagi2_flashnext_dots3_amd.dsa import PortableSparseImpl
    NQ, CTX, bs, K, H, ks = 2048, 65536, 64, 2048, 128, 0.8
    nblk, pad = CTX // bs, 8
    store = torch.empty(nblk, bs + pad, 576, dtype=torch.uint8, device=dev)
    g = torch.Generator(device=dev).manual_seed(3)
    for b0 in range(0, nblk, 256):
        n = min(256, nblk - b0)
        store[b0:b0 + n] = torch.randn(n, bs + pad, 576, generator=g, device=dev).to(torch.float8_e4m3fn) \
            .view(torch.uint8)
    cache = store[:, :bs]                                  # [nblk, bs, 576], block stride (bs + pad) rows
    gp = torch.Generator(device=dev).manual_seed(4)
    pos = torch.stack([torch.randperm(CTX, generator=gp, device=dev)[:K] for _ in range(NQ)])
    pos[5, ::4] = -1                                       # unused entries
    bt = torch.randperm(nblk, generator=torch.Generator().manual_seed(5)).to(dev)
    gidx = torch.where(pos >= 0, bt[pos.clamp(min=0) // bs] * (bs + pad) + pos.clamp(min=0) % bs,
                       torch.full_like(pos, -1))
    impl = PortableSparseImpl(H, 576, 192 ** -0.5, 1, None, None, "fp8", None, "decoder", None)
    q = torch.randn(NQ, H, 576, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16).to(dev)
    impl._run(q[:32], cache, gidx[:32], ks)                # first call: library load and the workspace reserve
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(dev)
    base = torch.cuda.memory_allocated(dev)
    print("[576] plugin paged cache, 2048 tokens x 2048 rows", flush=True)
    out = impl._run(q, cache, gidx, ks)
    torch.cuda.synchronize()
    added = torch.cuda.max_memory_allocated(dev) - base
    print(f"[576] memory added by the call: {added / 2**20:.0f} MiB", flush=True)
    assert added < 0.6 * 2**30
    tokens = [0, 5, 300, 777, 1024, 1500, 2000, NQ - 1]
    flat = store.view(-1, 576)
    sel = gidx[tokens]
    rows = flat[sel.clamp(min=0).reshape(-1)].cpu().numpy()
    local = np.where(sel.cpu().numpy() >= 0, np.arange(sel.numel()).reshape(sel.shape), -1)
    o_ref, l_ref = ref.attention(q[tokens].float().cpu().numpy(), rows, local, 192 ** -0.5, ks, fmt=576)
    o = out[tokens].float().cpu().numpy()
    assert attn_excess(o, o_ref) <= 0
