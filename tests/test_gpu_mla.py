"""GPU parity of the FP8 absorbed matmuls (spmla_bmm_fp8) and the fused decode query build (spmla_mla_query) vs the
fp64 oracle: fp32 accumulation of exact bf16 products, bounded by 2^-18 of sum |a w| per element (plus the bf16
output's own rounding); q_pe columns bit-exact."""
import numpy as np
import pytest
import torch

from oracle import spmla_ref as ref

pytestmark = pytest.mark.gpu


def _weights(N, J, K, scale_k, seed):
    g = torch.Generator().manual_seed(seed)
    codes = (torch.randn(N, J, K, generator=g) * 60).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
    sshape = (N, J, (K + 127) // 128) if scale_k else (N, K, (J + 127) // 128)
    scales = torch.exp(torch.randn(sshape, generator=g)) * 1e-3
    return codes, scales


def _bound(a, codes, scales, scale_k):
    W = ref.bmm_fp8_weights(codes.numpy(), scales.numpy(), scale_k)
    return np.einsum("nbk,njk->nbj", np.abs(a.float().numpy().astype(np.float64)), np.abs(W))


@pytest.mark.parametrize("scale_k,N,B,J,K,out_f32", [(False, 8, 64, 512, 128, True), (True, 8, 64, 128, 512, True),
                                                     (True, 4, 300, 200, 136, False), (False, 3, 37, 512, 128, False)])
def test_bmm_fp8(dev, scale_k, N, B, J, K, out_f32):
    from arcagi2_flashnext_dots3_amd import kernels
    codes, scales = _weights(N, J, K, scale_k, N + B)
    g = torch.Generator().manual_seed(7)
    a_t = torch.randn(B, N, K, generator=g).to(torch.bfloat16)            # [B, N, K] seen as [N, B, K]
    a = a_t.transpose(0, 1)
    print(f"[bmm_fp8] scale_k={scale_k} N={N} B={B} J={J} K={K}", flush=True)
    out = torch.empty(N, B, J, dtype=torch.float32 if out_f32 else torch.bfloat16, device=dev)
    kernels.bmm_fp8(a_t.to(dev).transpose(0, 1), codes.to(dev), scales.to(dev), scale_k, out)
    torch.cuda.synchronize()
    want = ref.bmm_fp8(a.float().numpy(), codes.numpy(), scales.numpy(), scale_k)
    bound = 2.0 ** -18 * _bound(a, codes, scales, scale_k) + (0.0 if out_f32 else 2.0 ** -8 * np.abs(want))
    got = out.float().cpu().numpy().astype(np.float64)
    assert np.all(np.abs(got - want) <= bound + 1e-30)


def test_mla_query(dev):
    """q[t, h, :512] = q_nope[t, h] @ W_UK_T[h] (bf16), q[t, h, 512:] = q_pe[t, h] bit for bit, written into a padded
    buffer (row strides larger than 576)."""
    from arcagi2_flashnext_dots3_amd import kernels
    T, H = 70, 16
    codes, scales = _weights(H, 512, 128, False, 11)
    g = torch.Generator().manual_seed(12)
    q_nope = torch.randn(T, H, 128, generator=g).to(torch.bfloat16)
    q_pe = torch.randn(T, H, 64, generator=g).to(torch.bfloat16)
    buf = torch.full((T, H, 640), 7, dtype=torch.bfloat16, device=dev)
    q = buf[:, :, :576]
    kernels.mla_query(q_nope.to(dev), q_pe.to(dev), codes.to(dev), scales.to(dev), out=q)
    torch.cuda.synchronize()
    a = q_nope.transpose(0, 1)
    want = ref.bmm_fp8(a.float().numpy(), codes.numpy(), scales.numpy(), False).transpose(1, 0, 2)
    bound = (2.0 ** -18 * _bound(a, codes, scales, False) + 2.0 ** -8 * np.abs(
        ref.bmm_fp8(a.float().numpy(), codes.numpy(), scales.numpy(), False))).transpose(1, 0, 2)
    got = q[:, :, :512].float().cpu().numpy()
    assert np.all(np.abs(got - want) <= bound + 1e-30)
    assert torch.equal(q[:, :, 512:].cpu(), q_pe)
    assert bool((buf[:, :, 576:] == 7).all())
