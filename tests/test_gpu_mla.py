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


@pytest.mark.parametrize("scale_k", [True, False])
def test_bmm_fp8_dequant_exact(dev, scale_k):
    """A = identity rows: C[n][b][j] = W[n][j][b] with nothing else added, so the fp32 output shows every dequantized
    weight bit for bit: all 254 non-NaN codes at scales that land on bf16 rounding ties and near the fp32 subnormal
    range."""
    from arcagi2_flashnext_dots3_amd import kernels
    N, J, K = 2, 256, 256
    c = np.arange(J * K, dtype=np.int64).reshape(1, J, K) * 7 % 256
    c = np.where((c & 0x7f) == 0x7f, 0, c).astype(np.uint8).repeat(N, 0)                 # no NaN codes
    g = np.random.default_rng(3)
    sshape = (N, J, 2) if scale_k else (N, K, 2)
    # 1 + 2^-8 + 2^-9 style scales give products with exact halfway bits; some tiny, some plain random
    ties = (1.0 + g.integers(0, 256, sshape) / 256.0 + 2.0 ** -9) * 2.0 ** g.integers(-20, 4, sshape)
    scales = np.where(g.random(sshape) < 0.5, ties, np.exp(g.standard_normal(sshape)) * 1e-3).astype(np.float32)
    scales[0, 0, 0] = 2.0 ** -110                      # tiny products, still normal (MFMA may flush subnormal inputs)
    a = torch.eye(K, dtype=torch.bfloat16).expand(N, K, K).contiguous()
    out = torch.empty(N, K, J, dtype=torch.float32, device=dev)
    kernels.bmm_fp8(a.to(dev), torch.from_numpy(c).to(dev), torch.from_numpy(scales).to(dev), scale_k, out)
    torch.cuda.synchronize()
    want = ref.bmm_fp8_weights(c, scales, scale_k).transpose(0, 2, 1)
    assert np.array_equal(out.cpu().numpy().astype(np.float64), want)


@pytest.mark.parametrize("out_f32", [True, False])
def test_bmm_fp8_strided_operands(dev, out_f32):
    """Operands the staged (LDS) kernel does not take — A strided along k, codes strided along k, an output strided
    along j — run on the register kernel; both kernels meet the same bound, and the staged one serves the same
    values with contiguous copies of the operands."""
    from arcagi2_flashnext_dots3_amd import kernels
    N, B, J, K = 3, 50, 96, 256
    codes, scales = _weights(N, J, K, True, 21)
    g = torch.Generator().manual_seed(22)
    a_nkb = torch.randn(N, K, B, generator=g).to(torch.bfloat16)
    a = a_nkb.transpose(1, 2)                                          # [N, B, K], stride along k = B
    codes_t = codes.transpose(1, 2).contiguous().transpose(1, 2)       # [N, J, K], stride along k = J
    dt = torch.float32 if out_f32 else torch.bfloat16
    out_s = torch.empty(N, J, B, dtype=dt, device=dev).transpose(1, 2)  # stride along j = B
    kernels.bmm_fp8(a_nkb.to(dev).transpose(1, 2), codes_t.to(dev), scales.to(dev), True, out_s)
    out_c = torch.empty(N, B, J, dtype=dt, device=dev)
    kernels.bmm_fp8(a.contiguous().to(dev), codes.to(dev), scales.to(dev), True, out_c)
    torch.cuda.synchronize()
    want = ref.bmm_fp8(a.float().numpy(), codes.numpy(), scales.numpy(), True)
    bound = 2.0 ** -18 * _bound(a, codes, scales, True) + (0.0 if out_f32 else 2.0 ** -8 * np.abs(want))
    for got in (out_s, out_c):
        assert np.all(np.abs(got.float().cpu().numpy().astype(np.float64) - want) <= bound + 1e-30)
