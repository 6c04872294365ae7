"""Pins of the oracle's FP8 absorbed matmul (against the torch statement of the reference's dequantization and a
python triple loop) and of the host-side weight conversion (exact round trip of block-FP8 weights). CPU only."""
import numpy as np
import torch

from oracle import spmla_ref as ref
from arcagi2_flashnext_dots3_amd import mla_fp8


def _weights(N, J, K, scale_k, seed):
    g = torch.Generator().manual_seed(seed)
    codes = (torch.randn(N, J, K, generator=g) * 60).clamp(-448, 448).to(torch.float8_e4m3fn)
    sshape = (N, J, (K + 127) // 128) if scale_k else (N, K, (J + 127) // 128)
    scales = torch.exp(torch.randn(sshape, generator=g)) * 1e-3
    return codes, scales


def test_bmm_fp8_oracle_vs_torch_and_loop():
    for scale_k in (True, False):
        N, B, J, K = 3, 5, 256, 384
        codes, scales = _weights(N, J, K, scale_k, 1)
        a = torch.randn(N, B, K, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
        if scale_k:
            S = scales.repeat_interleave(128, 2)[:, :, :K]
        else:
            S = scales.repeat_interleave(128, 2)[:, :, :J].transpose(1, 2)
        wb = (codes.float() * S).to(torch.bfloat16).double()          # the reference's dequantization (torch)
        want = torch.matmul(a.double(), wb.transpose(1, 2)).numpy()
        got = ref.bmm_fp8(a.float().numpy(), codes.view(torch.uint8).numpy(), scales.numpy(), scale_k)
        assert np.array_equal(ref.bmm_fp8_weights(codes.view(torch.uint8).numpy(), scales.numpy(), scale_k),
                              wb.numpy())
        assert np.allclose(got, want, rtol=0, atol=1e-9 * np.abs(want).max())
    # triple loop on a tiny case
    codes, scales = _weights(1, 2, 16, True, 3)
    a = torch.randn(1, 2, 16, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    got = ref.bmm_fp8(a.float().numpy(), codes.view(torch.uint8).numpy(), scales.numpy(), True)
    for b in range(2):
        for j in range(2):
            acc = 0.0
            for k in range(16):
                w = float((codes[0, j, k].float() * scales[0, j, 0]).to(torch.bfloat16))
                acc += float(a[0, b, k]) * w
            assert abs(got[0, b, j] - acc) <= 1e-12 * max(1.0, abs(acc))


def test_convert_round_trip():
    N, P, L, V = 4, 128, 512, 128
    g = torch.Generator().manual_seed(5)
    si = torch.exp(torch.randn((N * (P + V)) // 128, L // 128, generator=g)) * 1e-2
    rows = torch.arange(N * (P + V)) // 128
    full = si[rows][:, torch.arange(L) // 128]                       # [N (P + V), L]
    codes = (torch.randn(N * (P + V), L, generator=g) * 50).clamp(-448, 448).to(torch.float8_e4m3fn)
    kvb = (codes.float() * full).to(torch.bfloat16).view(N, P + V, L)  # vLLM's bf16 kv_b rows
    W_UK_T = kvb[:, :P, :].contiguous()                             # [N, P, L]
    W_UV = kvb[:, P:, :].transpose(1, 2).contiguous()               # [N, L, V]
    f = mla_fp8.convert(W_UK_T, W_UV, si)
    assert f is not None
    (cu, su, ku), (cv, sv, kv) = f
    assert cu.shape == (N, L, P) and su.shape == (N, P, L // 128) and not ku
    assert cv.shape == (N, V, L) and sv.shape == (N, V, L // 128) and kv
    # the dequantized FP8 forms equal the bf16 weights exactly
    wu = ref.bmm_fp8_weights(cu.numpy(), su.numpy(), False)          # [N, L, P]
    assert np.array_equal(wu, W_UK_T.transpose(1, 2).double().numpy())
    wv = ref.bmm_fp8_weights(cv.numpy(), sv.numpy(), True)           # [N, V, L]
    assert np.array_equal(wv, W_UV.transpose(1, 2).double().numpy())
    # a weight that no block scale reproduces is refused
    bad = W_UK_T.clone()
    bad[0, 0, 0] = bad[0, 0, 0] * 1.0078125 + 1e-3
    assert mla_fp8.convert(bad, W_UV, si) is None
