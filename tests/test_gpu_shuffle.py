"""GPU parity of the indexer key write into vLLM's paged SHUFFLE cache (bit-exact bytes vs the oracle) and of the
paged logits over it (vs the fp64 oracle within the logits tolerance, identical -inf pattern, next_n > 1 and 2-D
seq_lens; bit-identical to the 132-byte-row kernel on the same keys where no clamp applies)."""
import numpy as np
import pytest
import torch

from oracle import spmla_ref as ref
from tests.helpers import bf16_bits

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bs,ue8m0", [(64, False), (16, True), (128, False)])
def test_key_write_shuffle(dev, bs, ue8m0):
    from arcagi2_flashnext_dots3_amd import kernels
    nb, n = 7, 300
    g = torch.Generator().manual_seed(bs)
    k = torch.randn(n, 128, generator=g).to(torch.bfloat16) * torch.exp(torch.randn(n, 1, generator=g) * 2).to(torch.bfloat16)
    k[3] = 0
    slots = torch.randperm(nb * bs, generator=g)[:n].to(torch.int64)
    slots[::17] = -1
    slots[5] = nb * bs + 9
    cache = torch.full((nb, bs, 1, 132), 0xA5, dtype=torch.uint8, device=dev)
    print(f"[shuffle write] bs={bs} ue8m0={ue8m0}", flush=True)
    kernels.index_key_write_shuffle(k.to(dev), slots.to(dev), cache, ue8m0=ue8m0)
    torch.cuda.synchronize()
    exp = np.full((nb, bs * 132), 0xA5, dtype=np.uint8)
    ref.index_key_write_shuffle(bf16_bits(k), slots.numpy(), exp, bs, ue8m0=ue8m0)
    assert np.array_equal(cache.cpu().numpy().reshape(nb, -1), exp)


@pytest.mark.parametrize("B,nn,L,two_d", [(4, 1, 2048, False), (3, 3, 5000, False), (2, 2, 700, True)])
def test_paged_mqa_logits(dev, B, nn, L, two_d):
    from arcagi2_flashnext_dots3_amd import kernels
    bs = 64
    nbp = (L + bs - 1) // bs
    nb = B * nbp + 2
    g = torch.Generator().manual_seed(L)
    k = torch.randn(nb * bs, 128, generator=g).to(torch.bfloat16)
    rows = np.zeros((nb * bs, 132), dtype=np.uint8)
    ref.index_key_write(bf16_bits(k), np.arange(nb * bs), rows)
    cache = torch.from_numpy(ref.shuffle_layout(rows, bs)).to(dev).view(nb, bs, 1, 132)
    bt = torch.randperm(nb, generator=g)[: B * nbp].reshape(B, nbp).to(torch.int32)
    q = torch.randn(B, nn, 64, 128, generator=g).to(torch.bfloat16)
    w = torch.rand(B * nn, 64, generator=g)
    if two_d:
        sl = torch.randint(L // 2, L + 1, (B, nn), generator=g).to(torch.int32)
    else:
        sl = torch.randint(L // 2, L + 1, (B,), generator=g).to(torch.int32)
        sl[0] = L
    print(f"[paged logits] B={B} next_n={nn} L={L} 2d={two_d}", flush=True)
    out = kernels.paged_mqa_logits(q.to(dev), cache, w.to(dev), sl.to(dev), bt.to(dev), L)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    exp = ref.paged_mqa_logits(q.float().numpy(), ref.shuffle_layout(rows, bs), w.numpy(), sl.numpy(), bt.numpy(), bs, L)
    assert np.array_equal(np.isinf(got), np.isinf(exp))
    fin = np.isfinite(exp)
    err = np.abs(got[fin] - exp[fin]) / np.maximum(1.0, np.abs(exp[fin]))
    print(f"[paged logits] max rel err {err.max():.3e}", flush=True)
    assert err.max() <= 2e-5
    # the same keys as 132-byte rows through the shard kernel: identical bits (only the addressing differs)
    req, ctx = kernels.paged_ctx(sl.to(dev), nn)
    out2 = kernels.index_logits(q.reshape(B * nn, 64, 128).to(dev), w.to(dev),
                                torch.from_numpy(rows).to(dev).view(nb, bs, 132), bt.to(dev), bs, req, ctx, L)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)


def test_paged_logits_fp8_query(dev):
    """An e4m3 query (the reference's dtype) gives the logits of its exact bf16 widening."""
    from arcagi2_flashnext_dots3_amd import kernels
    bs, nb, B, L = 16, 8, 2, 100
    g = torch.Generator().manual_seed(3)
    rows = np.zeros((nb * bs, 132), dtype=np.uint8)
    ref.index_key_write(bf16_bits(torch.randn(nb * bs, 128, generator=g)), np.arange(nb * bs), rows)
    cache = torch.from_numpy(ref.shuffle_layout(rows, bs)).to(dev)
    q8 = (torch.randn(B, 1, 64, 128, generator=g) * 4).to(torch.float8_e4m3fn).to(dev)
    w = torch.rand(B, 64, generator=g).to(dev)
    bt = torch.arange(nb, dtype=torch.int32).reshape(B, nb // B).to(dev)
    sl = torch.tensor([L, 37], dtype=torch.int32, device=dev)
    a = kernels.paged_mqa_logits(q8, cache, w, sl, bt, L)
    b = kernels.paged_mqa_logits(q8.to(torch.bfloat16), cache, w, sl, bt, L)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_mqa_logits_flat(dev):
    """Prefill logits over a flat key gather [N, 128] + scales [N] with per-row [ks, ke) ranges vs the oracle."""
    from arcagi2_flashnext_dots3_amd import kernels
    N, M = 3000, 9
    g = torch.Generator().manual_seed(6)
    k = torch.randn(N, 128, generator=g).to(torch.bfloat16)
    rows = np.zeros((N, 132), dtype=np.uint8)
    ref.index_key_write(bf16_bits(k), np.arange(N), rows)
    codes = torch.from_numpy(rows[:, :128].copy())
    scales = torch.from_numpy(rows[:, 128:].copy().view(np.float32)[:, 0].copy())
    q = torch.randn(M, 64, 128, generator=g).to(torch.bfloat16)
    w = torch.rand(M, 64, generator=g)
    ks = torch.tensor([0, 0, 100, 2999, 500, 1000, 0, 64, 2048], dtype=torch.int32)
    ke = torch.tensor([3000, 1, 2100, 3000, 500, 2999, 257, 96, 3000], dtype=torch.int32)
    print("[mqa logits] flat", flush=True)
    out = kernels.mqa_logits(q.to(dev), (codes.to(dev).view(torch.float8_e4m3fn), scales.to(dev).view(N, 1)),
                             w.to(dev), ks.to(dev), ke.to(dev))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    exp = ref.mqa_logits(q.float().numpy(), rows[:, :128], rows[:, 128:].copy().view(np.float32)[:, 0], w.numpy(),
                         ks.numpy(), ke.numpy())
    assert np.array_equal(np.isinf(got), np.isinf(exp))
    fin = np.isfinite(exp)
    err = np.abs(got[fin] - exp[fin]) / np.maximum(1.0, np.abs(exp[fin]))
    print(f"[mqa logits] max rel err {err.max():.3e}", flush=True)
    assert err.max() <= 2e-5
