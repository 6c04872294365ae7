"""Seeded input generators shared by the tests and bench.py (synthetic data with the shapes of BASELINE.json's
configs), and the attention output bar. Nothing here computes a result: oracle/ does that."""
import numpy as np
import torch

D_LAT, D_ROPE, D_QK, ROW = 512, 64, 576, 656


def bf16_bits(x):
    """float tensor -> numpy uint16 bf16 bit patterns (round to nearest even, torch's conversion)."""
    return torch.as_tensor(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def make_pool_656(R, seed=1, scale=1.0, device=None):
    """R Row656 rows from N(0, scale^2) latent / rope (bf16), packed by the oracle's writer. Returns
    (pool uint8 numpy [R, 656], kv bits [R, 512], pe bits [R, 64])."""
    from oracle import spmla_ref as ref
    g = torch.Generator().manual_seed(seed)
    kv = bf16_bits(torch.randn(R, D_LAT, generator=g) * scale)
    pe = bf16_bits(torch.randn(R, D_ROPE, generator=g) * scale)
    pool = np.zeros((R, ROW), dtype=np.uint8)
    ref.cache_write_656(kv, pe, np.arange(R), pool)
    return pool, kv, pe


def make_pool_576(R, seed=1, scale=1.0, kv_scale=1.0):
    """R Row576 rows (the per-tensor fp8 cache) from N(0, scale^2) latent / rope, written by the oracle's writer with
    kv_scale. Returns pool uint8 numpy [R, 576]."""
    from oracle import spmla_ref as ref
    g = torch.Generator().manual_seed(seed)
    kv = bf16_bits(torch.randn(R, D_LAT, generator=g) * scale)
    pe = bf16_bits(torch.randn(R, D_ROPE, generator=g) * scale)
    pool = np.zeros((R, D_QK), dtype=np.uint8)
    ref.cache_write_576(kv, pe, np.arange(R), pool, kv_scale)
    return pool


def make_q(T, H, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(T, H, D_QK, generator=g) * scale).to(torch.bfloat16)


def distinct_idx(T, K, R, seed=2):
    g = torch.Generator().manual_seed(seed)
    return torch.stack([torch.randperm(R, generator=g)[:K] for _ in range(T)]).to(torch.int32)


def half_ulp_bf16(x):
    """Half a bf16 ulp of |x| (2^(e - 8) for |x| in [2^e, 2^(e + 1))), 0 for x = 0."""
    a = np.abs(np.asarray(x, dtype=np.float64))
    e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    return np.where(a > 0, 2.0 ** (e - 8), 0.0)


def attn_excess(o, o_ref, tol=1e-2):
    """Largest amount by which |o - o_ref| exceeds the attention output bar tol + half a bf16 ulp of o_ref (the
    rounding of the bf16 output itself); <= 0 passes."""
    o, o_ref = np.asarray(o, dtype=np.float64), np.asarray(o_ref, dtype=np.float64)
    return float((np.abs(o - o_ref) - (tol + half_ulp_bf16(o_ref))).max()) if o.size else 0.0
