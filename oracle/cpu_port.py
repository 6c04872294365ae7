"""float32 torch-CPU restatement of the sparse-MLA decode step, timed as bench.py's CPU baseline (kind "port").
TEST / BASELINE INFRASTRUCTURE ONLY.

It is the reference's own torch statement of the path (dotsnote/kaggle/runtime_dataset/bench_offload_attn2.py:77-93:
gather the rows, einsum q . row, base-2 masked softmax, p . V / sum p; LSE as in
dotsnote/engine/vllm_patch/vllm/v1/attention/ops/xpu_mla_sparse.py:155-161), written with batched matmuls and run on
the host cores in fp32.
"""
import os

import torch

_E4M3 = None


def _e4m3_table():
    global _E4M3
    if _E4M3 is None:
        _E4M3 = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float()
    return _E4M3


def threads():
    return len(os.sched_getaffinity(0))


def dequant_rows_656(rows_u8):
    """[..., 656] uint8 -> latent [..., 512] fp32, rope [..., 64] fp32"""
    tab = _e4m3_table()
    codes = tab[rows_u8[..., :512].long()]
    sc = rows_u8[..., 512:528].contiguous().view(torch.float32)
    lat = (codes.view(*codes.shape[:-1], 4, 128) * sc.unsqueeze(-1)).view(*codes.shape[:-1], 512)
    rope = rows_u8[..., 528:656].contiguous().view(torch.bfloat16).float()
    return lat, rope


def attention_f32(q, pool, idx, sm_scale, kv_scale=1.0):
    """q [T, H, 576] bf16/fp32 (CPU), pool [R, 656] uint8 (CPU), idx [T, K] int32 -> out [T, H, 512] fp32, lse [T, H]."""
    R = pool.shape[0]
    valid = (idx >= 0) & (idx < R)
    rows = pool[idx.clamp(0, R - 1).long()]                         # [T, K, 656]
    lat, rope = dequant_rows_656(rows)
    k = torch.cat([lat, rope], -1)                                 # [T, K, 576]
    s = torch.bmm(q.float(), k.transpose(1, 2)) * (sm_scale * kv_scale * 1.4426950408889634)
    s = s.masked_fill(~valid[:, None, :], -1e30)
    m = s.amax(-1, keepdim=True)
    p = torch.exp2(s - m) * valid[:, None, :]
    l = p.sum(-1, keepdim=True)
    o = torch.bmm(p, lat) / l.clamp_min(1e-30) * kv_scale
    lse = (m + torch.log2(l)) * 0.6931471805599453
    return o, lse.squeeze(-1)
