"""GPU parity of the cache / key writers: FP8 codes, scales and rope bytes bit-exact vs the oracle."""
import numpy as np
import pytest
import torch

from oracle import spmla_ref as ref
from tests.helpers import bf16_bits

pytestmark = pytest.mark.gpu


def _inputs(n, seed, special=True):
    g = torch.Generator().manual_seed(seed)
    kv = torch.randn(n, 512, generator=g) * torch.exp(torch.randn(n, 1, generator=g) * 3)
    pe = torch.randn(n, 64, generator=g)
    if special and n >= 8:
        kv[0] = 0.0                                       # zero row: scale floor 1e-12
        kv[1, :128] = 0.0                                 # one zero group
        kv[2, 5] = 448.0 * 4                              # amax exactly 448 * 2^k in group 0
        kv[3] = -kv[3]
        kv[4, 128:256] = 1e-30                            # denormal-scale group
        kv[5] = torch.where(kv[5] > 0, 2.0 ** -8, -(2.0 ** -8))
    return kv.to(torch.bfloat16), pe.to(torch.bfloat16)


@pytest.mark.parametrize("n,R,seed", [(64, 128, 0), (8192, 20000, 1)])
def test_cache_write_656(dev, n, R, seed):
    from arcagi2_flashnext_dots3_amd import kernels
    kv, pe = _inputs(n, seed)
    g = torch.Generator().manual_seed(seed + 100)
    slots = torch.randperm(R, generator=g)[:n].to(torch.int64)
    slots[::17] = -1                                      # padding slots are skipped
    print(f"[write656] n={n} R={R}", flush=True)
    cache = torch.full((R, 656), 0xAB, dtype=torch.uint8, device=dev)
    kernels.cache_write(kv.to(dev), pe.to(dev), slots.to(dev), cache)
    exp = np.full((R, 656), 0xAB, dtype=np.uint8)
    ref.cache_write_656(bf16_bits(kv), bf16_bits(pe), slots.numpy(), exp)
    got = cache.cpu().numpy()
    assert np.array_equal(got, exp)


def test_cache_write_paged_656(dev):
    # paged cache with a padded block stride (blocks of 64 rows, 64 spare bytes after each block)
    from arcagi2_flashnext_dots3_amd import kernels
    n, nb, bs = 300, 16, 64
    kv, pe = _inputs(n, 5)
    slots = torch.randperm(nb * bs, generator=torch.Generator().manual_seed(3))[:n].to(torch.int64)
    base = torch.zeros(nb, bs * 656 + 64, dtype=torch.uint8, device=dev)
    cache = base.as_strided((nb, bs, 656), (bs * 656 + 64, 656, 1))
    kernels.cache_write(kv.to(dev), pe.to(dev), slots.to(dev), cache)
    exp = np.zeros((nb * bs, 656), dtype=np.uint8)
    ref.cache_write_656(bf16_bits(kv), bf16_bits(pe), slots.numpy(), exp)
    got = base[:, : bs * 656].reshape(nb * bs, 656).cpu().numpy()
    assert np.array_equal(got, exp)
    assert int(base[:, bs * 656:].abs().sum() if base.dtype != torch.uint8 else base[:, bs * 656:].sum()) == 0


def test_cache_write_576(dev):
    from arcagi2_flashnext_dots3_amd import kernels
    n, R = 500, 1024
    kv, pe = _inputs(n, 9, special=False)
    kv = (kv.float() * 100).to(torch.bfloat16)            # values beyond 448: clamped
    slots = torch.randperm(R, generator=torch.Generator().manual_seed(4))[:n].to(torch.int64)
    cache = torch.zeros(R, 576, dtype=torch.uint8, device=dev)
    kernels.cache_write(kv.to(dev), pe.to(dev), slots.to(dev), cache, fmt=1, kv_scale=2.0)
    exp = np.zeros((R, 576), dtype=np.uint8)
    ref.cache_write_576(bf16_bits(kv), bf16_bits(pe), slots.numpy(), exp, kv_scale=2.0)
    assert np.array_equal(cache.cpu().numpy(), exp)


@pytest.mark.parametrize("ue8m0", [False, True])
def test_index_key_write(dev, ue8m0):
    from arcagi2_flashnext_dots3_amd import kernels
    n, R = 2000, 4096
    g = torch.Generator().manual_seed(21)
    k = (torch.randn(n, 128, generator=g) * torch.exp(torch.randn(n, 1, generator=g) * 4)).to(torch.bfloat16)
    k[0] = 0
    slots = torch.randperm(R, generator=g)[:n].to(torch.int64)
    store = torch.zeros(R, 132, dtype=torch.uint8, device=dev)
    kernels.index_key_write(k.to(dev), slots.to(dev), store, ue8m0=ue8m0)
    exp = np.zeros((R, 132), dtype=np.uint8)
    ref.index_key_write(bf16_bits(k), slots.numpy(), exp, ue8m0=ue8m0)
    assert np.array_equal(store.cpu().numpy(), exp)
