"""GPU parity of the compact Row400 host-row path: the encoder (spmla_cache_write fmt 2) and the decoding gathers
bit-exact vs the oracle; LayerOffload with compact host rows vs the oracle attention over the decoded rows."""
import numpy as np
import pytest
import torch

from oracle import spmla_ref as ref
from tests.helpers import bf16_bits, distinct_idx, make_q

pytestmark = pytest.mark.gpu


def _inputs(n, seed):
    """Latent values over a wide range per 32-value block, plus blocks that hit the quantizer's special cases."""
    g = torch.Generator().manual_seed(seed)
    kv = torch.randn(n, 512, generator=g) * torch.exp(torch.randn(n, 16, generator=g) * 3).repeat_interleave(32, 1)
    pe = torch.randn(n, 64, generator=g) * 4
    if n >= 8:
        kv[0] = 0.0                                          # zero blocks: k = -126
        kv[1, :32] = 1000.0                                  # clamps to 448: k = 6
        kv[1, 32:64] = -7.0                                  # amax / 7 == 1: k = 0
        kv[2, :32] = torch.tensor([(i % 16) * 0.125 for i in range(32)])   # ties of the grid
        kv[2, 31] = 7.0
        kv[3, :64] = 1e-30                                   # tiny blocks (k near -100)
        kv[4] = -kv[4]
        pe[5] = 1000.0                                       # rope clamps to 448
    return kv.to(torch.bfloat16), pe.to(torch.bfloat16)


def _oracle_rows(kv, pe, slots, R, kv_scale, fill):
    exp = np.full((R, 400), fill, dtype=np.uint8)
    ref.cache_write_400(bf16_bits(kv), bf16_bits(pe), slots, exp, kv_scale=kv_scale)
    return exp


@pytest.mark.parametrize("n,R,kv_scale", [(64, 100, 1.0), (4096, 9000, 0.37), (300, 300, 2.5)])
def test_cache_write_400(dev, n, R, kv_scale):
    from arcagi2_flashnext_dots3_amd import kernels
    kv, pe = _inputs(n, n)
    slots = torch.randperm(R, generator=torch.Generator().manual_seed(9))[:n].to(torch.int64)
    slots[::13] = -1
    print(f"[write400] n={n} R={R} kv_scale={kv_scale}", flush=True)
    cache = torch.full((R, 400), 0x5C, dtype=torch.uint8, device=dev)
    kernels.cache_write(kv.to(dev), pe.to(dev), slots.to(dev), cache, fmt=2, kv_scale=kv_scale)
    exp = _oracle_rows(kv, pe, slots.numpy(), R, kv_scale, 0x5C)
    got = cache.cpu().numpy()
    bad = np.nonzero((got != exp).any(1))[0]
    assert bad.size == 0, (bad[:5], np.nonzero(got[bad[0]] != exp[bad[0]]) if bad.size else None)


def test_cache_write_400_pinned_host(dev):
    """The encoder writing straight into pinned host memory (the compact host pool)."""
    from arcagi2_flashnext_dots3_amd import kernels
    n, R = 200, 512
    kv, pe = _inputs(n, 11)
    slots = torch.arange(n, dtype=torch.int64) * 2
    host = torch.zeros((R, 400), dtype=torch.uint8).pin_memory()
    kernels.cache_write(kv.to(dev), pe.to(dev), slots.to(dev), host, fmt=2, kv_scale=1.0)
    torch.cuda.synchronize()
    assert np.array_equal(host.numpy(), _oracle_rows(kv, pe, slots.numpy(), R, 1.0, 0))


@pytest.mark.parametrize("width,pinned", [(576, False), (656, False), (656, True), (576, True)])
def test_row400_gather(dev, width, pinned):
    from arcagi2_flashnext_dots3_amd import kernels
    n, R = 700, 1000
    kv, pe = _inputs(n, 2)
    src_np = _oracle_rows(kv, pe, np.arange(n), R, 0.5, 0)
    src_np[n:] = np.random.default_rng(1).integers(0, 256, (R - n, 400))          # arbitrary bytes decode too
    src = torch.from_numpy(src_np)
    src = src.pin_memory() if pinned else src.to(dev)
    rows = np.random.default_rng(3).integers(-3, R + 3, 3000)
    out = torch.full((3000, width), 7, dtype=torch.uint8, device=dev)
    print(f"[row400_gather] width={width} pinned={pinned}", flush=True)
    kernels.row400_gather(src, torch.from_numpy(rows).to(dev), out, pcie=pinned)
    exp = ref.row400_gather(src_np, rows, fmt=width)
    assert np.array_equal(out.cpu().numpy(), exp)


def test_row400_copy(dev):
    from arcagi2_flashnext_dots3_amd import kernels
    n, R, C = 256, 400, 128
    kv, pe = _inputs(n, 4)
    src_np = _oracle_rows(kv, pe, np.arange(n), R, 1.0, 0)
    g = np.random.default_rng(5)
    src_rows = g.integers(-2, R + 2, 500)
    dst_rows = g.integers(-2, C + 2, 500)
    # one writer per destination line (the kernel's order between duplicate destinations is not defined)
    _, first = np.unique(dst_rows, return_index=True)
    keep = np.zeros(500, bool)
    keep[first] = True
    src_rows, dst_rows = src_rows[keep], dst_rows[keep]
    dst = torch.full((C, 656), 3, dtype=torch.uint8, device=dev)
    kernels.row400_copy(torch.from_numpy(src_np).to(dev), torch.from_numpy(src_rows).to(dev), dst,
                        torch.from_numpy(dst_rows).to(dev))
    exp = np.full((C, 656), 3, dtype=np.uint8)
    for s, d in zip(src_rows, dst_rows):
        if 0 <= s < R and 0 <= d < C:
            exp[d] = ref.row400_gather(src_np, [s], fmt=656)[0]
    assert np.array_equal(dst.cpu().numpy(), exp)


@pytest.mark.parametrize("T,K,zero0", [(5, 64, False), (3, 2048, True), (1100, 8, False)])
def test_row400_gather_tiers(dev, T, K, zero0):
    from arcagi2_flashnext_dots3_amd import kernels
    g = np.random.default_rng(7)
    R = 3000
    host_np = g.integers(0, 256, (R, 400)).astype(np.uint8)
    host = torch.from_numpy(host_np).pin_memory()
    rows = g.integers(-2, R + 2, (T, K)).astype(np.int32)
    counts = g.integers(-1, K + 3, T).astype(np.int32)
    counts[0] = 0 if zero0 else K
    out = torch.full((T * K, 656), 9, dtype=torch.uint8, device=dev)
    kernels.row400_gather_tiers(host, torch.from_numpy(rows).to(dev), torch.from_numpy(counts).to(dev), out)
    torch.cuda.synchronize()
    exp = np.full((T * K, 656), 9, dtype=np.uint8)
    for t in range(T):
        c = min(max(int(counts[t]), 0), K)
        if c:
            exp[t * K:t * K + c] = ref.row400_gather(host_np, rows[t, :c], fmt=656)
    if zero0:
        exp[0] = 0
    assert np.array_equal(out.cpu().numpy(), exp)


@pytest.mark.parametrize("C,cache_fmt", [(0, "row656"), (300, "row656"), (300, "e2m2")])
def test_layer_offload_compact_rows(dev, C, cache_fmt):
    """store -> (hot set) -> attend with compact host rows: attention over the decoded Row576 values, kv_scale applied
    at both ends, vs the oracle; gather returns the reference's Row576 rows byte for byte. cache_fmt e2m2: the hot
    lines stay compact Row400 rows in HBM (the stored bytes themselves, write-through included)."""
    from arcagi2_flashnext_dots3_amd.sparse_offload import LayerOffload
    R, T, H, K, kv_scale = 1200, 3, 32, 256, 0.5
    g = torch.Generator().manual_seed(21)              # O(1) rows (the codec's edge cases are covered above)
    kv = (torch.randn(R, 512, generator=g) * torch.exp(torch.randn(R, 16, generator=g) * 0.5).repeat_interleave(32, 1)
          ).to(torch.bfloat16)
    pe = torch.randn(R, 64, generator=g).to(torch.bfloat16)
    lo = LayerOffload(R, dev, key="l0", cache_rows=C, row_fmt="e2m2", cache_fmt=cache_fmt)
    slots = torch.arange(R, dtype=torch.int64, device=dev)
    lo.store(kv.to(dev), pe.to(dev), slots, kv_scale=kv_scale)
    if C:
        lo.set_hot_rows(torch.arange(0, 2 * C, 2, dtype=torch.int64))
        lo.store(kv[:50].to(dev), pe[:50].to(dev), slots[:50], kv_scale=kv_scale)   # write-through of cached rows
    torch.cuda.synchronize()
    host_np = _oracle_rows(kv, pe, np.arange(R), R, kv_scale, 0)
    assert np.array_equal(lo.host.numpy(), host_np)
    rows576 = ref.row400_gather(host_np, np.arange(R), fmt=576)
    if C and cache_fmt == "e2m2":
        assert np.array_equal(lo.cache[:C].cpu().numpy(), host_np[np.arange(0, 2 * C, 2)])
    elif C:
        assert np.array_equal(lo.cache[:C].cpu().numpy(), ref.row400_gather(host_np, np.arange(0, 2 * C, 2), fmt=656))
    g = torch.full((10, 576), 1, dtype=torch.uint8, device=dev)
    lo.gather(torch.tensor([5, -1, 7, R, 0, 1199, 3, 2, 1, 4], device=dev), g)
    assert np.array_equal(g.cpu().numpy(), ref.row400_gather(host_np, [5, -1, 7, R, 0, 1199, 3, 2, 1, 4], fmt=576))
    q = make_q(T, H, seed=3)
    idx = distinct_idx(T, K, R, seed=4)
    idx[1, 100:] = -1
    sm = 1.0 / np.sqrt(192.0)
    out, lse = lo.attend(q.to(dev), idx.to(dev), sm, kv_scale, return_lse=True)
    eo, el = ref.attention(q.float().numpy(), rows576, idx.numpy(), sm, kv_scale, fmt=576)
    # bf16 output: 1e-2 absolute plus its own rounding (2^-9 relative)
    assert np.all(np.abs(out.float().cpu().numpy() - eo) <= 1e-2 + 2.0 ** -9 * np.abs(eo))
    assert np.abs(lse.cpu().numpy() - el).max() < 1e-3
    if C and cache_fmt == "e2m2":
        # same values as Row656 lines (the compact lines' hot tier is attended from Row576 staging, the Row656
        # lines' from the lines themselves: the two kernels differ only in fp32 summation order)
        lo2 = LayerOffload(R, dev, key="l1", cache_rows=C, row_fmt="e2m2")
        lo2.host.copy_(lo.host)
        lo2.set_hot_rows(torch.arange(0, 2 * C, 2, dtype=torch.int64))
        o2, l2 = lo2.attend(q.to(dev), idx.to(dev), sm, kv_scale, return_lse=True)
        torch.cuda.synchronize()
        err = (out.float() - o2.float()).abs() / o2.float().abs().clamp_min(1.0)
        assert float(err.max()) <= 1e-2 and float((lse - l2).abs().max()) <= 1e-4


@pytest.mark.parametrize("width,with_counts", [(576, True), (656, True), (576, False)])
def test_row400_decode_tiers(dev, width, with_counts):
    """Compact lines in HBM decoded per token list (spmla_row400_decode_tiers): out row t * K + k = the oracle's decode
    of src row rows[t, k] for k < counts[t] (every k without counts; invalid rows give zero rows), other out rows
    untouched; wide-range blocks, special blocks and arbitrary bytes decode as the oracle does."""
    from arcagi2_flashnext_dots3_amd import kernels
    n, R, T, K = 700, 1000, 5, 300
    kv, pe = _inputs(n, 7)
    src_np = _oracle_rows(kv, pe, np.arange(n), R, 0.5, 0)
    src_np[n:] = np.random.default_rng(8).integers(0, 256, (R - n, 400))
    src = torch.from_numpy(src_np).to(dev)
    g = np.random.default_rng(9)
    rows = g.integers(-2, R + 2, (T, K)).astype(np.int32)
    counts = np.array([K, 0, 17, 299, 150], dtype=np.int32)
    out = torch.full((T * K, width), 0xA5, dtype=torch.uint8, device=dev)
    print(f"[decode_tiers] width={width} counts={with_counts}", flush=True)
    kernels.row400_decode_tiers(src, torch.from_numpy(rows).to(dev),
                                torch.from_numpy(counts).to(dev) if with_counts else None, out)
    got = out.cpu().numpy()
    for t in range(T):
        c = counts[t] if with_counts else K
        exp = ref.row400_gather(src_np, rows[t, :c], fmt=width)
        assert np.array_equal(got[t * K:t * K + c], exp), t
        assert np.all(got[t * K + c:(t + 1) * K] == 0xA5)
