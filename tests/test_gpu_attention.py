"""GPU parity of spmla_attn_splitk / spmla_lse_merge against the CPU oracle (fp64), through the C-ABI.
Tolerances (north star): |out - ref| <= 1e-2 + half a bf16 ulp of ref (the rounding of the bf16 output itself) on
every element, max |lse - ref| <= 1e-3 against the fp64 oracle."""
import numpy as np
import pytest
import torch

from oracle import spmla_ref as ref
from tests.helpers import attn_excess, distinct_idx, make_pool_656, make_q

pytestmark = pytest.mark.gpu
OUT_TOL, LSE_TOL = 1e-2, 1e-3


def _check(dev, T, H, R, K, idx=None, split=1, kcount=None, seed=0, sm_scale=192 ** -0.5, qscale=1.0, pool=None):
    from arcagi2_flashnext_dots3_amd import kernels
    if pool is None:
        pool, _, _ = make_pool_656(R, seed=seed + 1)
    q = make_q(T, H, seed=seed, scale=qscale)
    if idx is None:
        idx = distinct_idx(T, K, R, seed=seed + 2)
    print(f"[attn] T={T} H={H} R={R} K={K} split={split} kcount={kcount is not None}", flush=True)
    qd = q.to(dev)
    out, lse = kernels.attend(qd, torch.from_numpy(pool).to(dev), idx.to(dev), sm_scale, split=split,
                              kcount=None if kcount is None else kcount.to(dev))
    torch.cuda.synchronize()
    o_ref, l_ref = ref.attention(q.float().numpy(), pool, idx.numpy(), sm_scale,
                                 kcount=None if kcount is None else kcount.numpy())
    o = out.float().cpu().numpy()
    l = lse.cpu().numpy()
    fin = np.isfinite(l_ref)
    assert np.array_equal(fin, np.isfinite(l)), "lse -inf pattern differs"
    err_o = attn_excess(o, o_ref, OUT_TOL)
    err_l = np.abs(l[fin] - l_ref[fin]).max() if fin.any() else 0.0
    print(f"[attn] max|o-ref| {np.abs(o - o_ref).max():.3e} (excess over the bar {err_o:.3e}) max|lse-ref| "
          f"{err_l:.3e} max|ref| {np.abs(o_ref).max():.2f}", flush=True)
    assert err_o <= 0 and err_l <= LSE_TOL
    assert np.all(o[~fin] == 0)
    return err_o, err_l


def test_config1_shape(dev):
    # B=1, 16 heads, 4096 rows, top-256 distinct, scale 1/sqrt(192)
    _check(dev, T=1, H=16, R=4096, K=256)


def test_decode_128_heads(dev):
    _check(dev, T=8, H=128, R=8192, K=2048, seed=3)


def test_split_merge(dev):
    _check(dev, T=4, H=64, R=4096, K=2048, split=4, seed=5)


def test_ragged_invalid_and_duplicates(dev):
    T, K, R = 6, 512, 2048
    g = torch.Generator().manual_seed(7)
    idx = torch.randint(0, R, (T, K), generator=g).to(torch.int32)        # duplicates allowed (counted twice)
    u = torch.rand(T, K, generator=g)
    idx[u < 0.1] = -1
    idx[(u >= 0.1) & (u < 0.15)] = R + 5                                    # out of range -> invalid
    idx[2, :] = -1                                                          # no valid entry: o = 0, lse = -inf
    idx[3, 100:] = -1
    _check(dev, T=T, H=32, R=R, K=K, idx=idx, seed=7)


def test_kcount_and_partial_tile(dev):
    T, K, R = 3, 200, 1000                                                  # K not a multiple of 32
    kc = torch.tensor([200, 37, 0], dtype=torch.int32)
    _check(dev, T=T, H=48, R=R, K=K, kcount=kc, seed=9)


def test_large_query_scale(dev):
    _check(dev, T=2, H=32, R=4096, K=1024, seed=11, qscale=30.0)


def test_attend_merge_two_tiers(dev):
    """spmla_attn_merge: the second tier's attention merged with the first tier's fp32 partial in the epilogue equals
    attention over the union of both tiers' rows (fp64 oracle) and the two-partial lse_merge; tokens with an empty
    tier (and one with both empty) included."""
    from arcagi2_flashnext_dots3_amd import kernels
    T, H, R, K = 6, 128, 3000, 512
    pool, _, _ = make_pool_656(R, seed=9)
    q = make_q(T, H, seed=8)
    idx = distinct_idx(T, K, R, seed=7)
    a = idx.clone()
    b = idx.clone()
    a[:, K // 3:] = -1                                     # tier A: the first third of each token's rows
    b[:, :K // 3] = -1                                     # tier B: the rest
    a[1] = -1                                              # token 1: tier A empty
    b[2] = -1                                              # token 2: tier B empty
    a[3] = -1
    b[3] = -1                                              # token 3: both empty
    union = torch.where(a >= 0, a, b)
    sm = 192 ** -0.5
    pd = torch.from_numpy(pool).to(dev)
    qd = q.to(dev)
    op, lp = kernels.attend_partial(qd, pd, a.to(dev), sm, 0.75)
    out, lse = kernels.attend_merge(qd, pd, b.to(dev), sm, 0.75, op[0], lp[0])
    op2, lp2 = kernels.attend_partial(qd, pd, b.to(dev), sm, 0.75)
    o_m, l_m = kernels.lse_merge(torch.cat([op, op2]), torch.cat([lp, lp2]))
    torch.cuda.synchronize()
    o_ref, l_ref = ref.attention(q.float().numpy(), pool, union.numpy(), sm, 0.75)
    o, l = out.float().cpu().numpy(), lse.cpu().numpy()
    fin = np.isfinite(l_ref)
    assert np.array_equal(fin, np.isfinite(l)) and not fin[3].any() and np.all(o[3] == 0)
    assert attn_excess(o, o_ref, OUT_TOL) <= 0
    assert np.abs(l[fin] - l_ref[fin]).max() <= LSE_TOL
    assert np.abs(o - o_m.float().cpu().numpy()).max() <= 2.0 ** -7 * max(1.0, np.abs(o).max())
    assert np.abs(l[fin] - l_m.cpu().numpy()[fin]).max() <= 1e-5


def test_nan_row_zero_is_never_read(dev):
    """Invalid entries (-1, out of range, past kcount) read the kernel's own zero row, not row 0 of the pool: with
    row 0 set to NaN codes, scales and rope, and never selected, outputs and lse stay finite and equal the oracle."""
    T, H, R, K = 3, 64, 2048, 512
    pool, _, _ = make_pool_656(R, seed=13)
    pool[0, :] = 0xFF                                      # e4m3 NaN codes, NaN scales and rope
    g = torch.Generator().manual_seed(14)
    idx = (torch.randperm(R - 1, generator=g)[:T * K] + 1).view(T, K).to(torch.int32)   # row 0 never selected
    idx[0, ::3] = -1
    idx[1, 100:] = R + 7
    kc = torch.tensor([K, K, 37], dtype=torch.int32)
    _check(dev, T=T, H=H, R=R, K=K, idx=idx, kcount=kc, seed=14, pool=pool)
