"""Pins of the oracle's Row400 (compact e2m2b32 host row) codec, independent of its own formulas: a float64 brute
force over the 16-point e2m2 grid, the byte layout written out position by position, exactness against the e4m3
decoder, and the decode path checked against the Row576 writer. CPU only."""
import numpy as np
import torch

from oracle import spmla_ref as ref
from tests.helpers import bf16_bits

# the e2m2 grid in units of 2^k: magnitude index (e2 << 2) | m -> (e2 ? 4 + m : m) * 2^(max(e2, 1) - 3)
GRID = np.array([(((i >> 2) and 4 + (i & 3)) or (i & 3)) * 2.0 ** (max(i >> 2, 1) - 3) for i in range(16)])


def _brute(x):
    """float64 brute force of the quantizer on one row of 512 fp32 values -> (codes, k)."""
    codes = np.zeros(512, dtype=np.int64)
    ks = np.zeros(16, dtype=np.int64)
    for b in range(16):
        blk = x[32 * b:32 * b + 32].astype(np.float64)
        r = float(np.float32(np.float32(np.abs(x[32 * b:32 * b + 32]).max()) / np.float32(7.0)))  # IEEE fp32 divide
        if r < 2.0 ** -126:
            k = -126
        else:
            k = next(k for k in range(-126, 128) if r <= 2.0 ** k)
        ks[b] = k
        for j, v in enumerate(blk):
            y = abs(v) * 2.0 ** -k
            best, bd = 0, None
            for m in range(16):                      # nearest grid point; ties -> the larger magnitude
                d = abs(y - GRID[m])
                if bd is None or d <= bd:
                    best, bd = m, d
            codes[32 * b + j] = best | (16 if (v < 0 and best > 0) else 0)
    return codes, ks


def _rows(n, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, 512, generator=g) * torch.exp(torch.randn(n, 16, generator=g) * 3).repeat_interleave(32, 1)
    x = x.clamp(-448, 448)
    x[0] = 0
    x[1, :32] = 448.0
    x[1, 32:64] = -7.0                                # amax / 7 == 1 exactly: k = 0, -7 -> magnitude 15
    x[1, 64:96] = 2.0 ** -140                         # fp32 subnormal block: k = -126
    x[1, 96:128] = torch.linspace(-1, 1, 32) * 7 * 2.0 ** -20
    x[2, :32] = torch.tensor([(i % 16) * 0.125 for i in range(32)])    # odd multiples: ties of the y < 2 grids
    x[2, 31] = 7.0
    x[3, :16] = torch.tensor([2.25, 2.75, 3.25, 3.75, 4.5, 5.5, 6.5, 7.0, -2.25, -4.5, -6.5, 0.375, -0.125, 1.875, 3.9, 7.4])
    x[3, 16:32] = 0.0
    return x.to(torch.float32).numpy()


def test_row400_quant_brute_force():
    x = _rows(24, 0)
    code, k = ref.row400_quant(x)
    for i in range(x.shape[0]):
        bc, bk = _brute(x[i])
        assert np.array_equal(k[i], bk), i
        assert np.array_equal(code[i], bc), (i, np.nonzero(code[i] != bc))


def test_row400_quant_hand_examples():
    x = np.zeros((1, 512), dtype=np.float32)
    x[0, :32] = 1.0
    x[0, 0] = 448.0                                   # 448 / 7 = 64: k = 6, 448 -> magnitude 15 (7 * 64)
    x[0, 32:64] = 0.0
    x[0, 64] = 7.0000005                              # fp32(7.0000005 / 7) > 1: k = 1
    x[0, 96] = 7.0                                    # block max 7: k = 0, y = 0.125 -> 4y + 0.5 = 1: magnitude 1
    x[0, 97] = 0.125
    x[0, 98] = np.float32(0.125) - np.float32(2.0 ** -27)   # 4y + 0.5 = 1 - 2^-25 rounds to 1.0 in fp32: magnitude 1
    x[0, 99] = -0.0
    x[0, 100] = -0.1                                  # magnitude 0 after rounding: no sign bit
    x[0, 101] = -0.15                                 # nearest 0.25: magnitude 1 with sign
    code, k = ref.row400_quant(x)
    assert k[0, 0] == 6 and code[0, 0] == 15 and code[0, 1] == 0     # 1.0 / 64 = 0.0156 -> 0
    assert k[0, 1] == -126 and np.all(code[0, 32:64] == 0)
    assert k[0, 2] == 1
    assert k[0, 3] == 0 and code[0, 96] == 15 and code[0, 97] == 1 and code[0, 98] == 1
    assert code[0, 99] == 0 and code[0, 100] == 0 and code[0, 101] == 17


def test_row400_layout():
    N = 2
    code = np.arange(N * 512).reshape(N, 512) * 7 % 32
    k = np.arange(N * 16).reshape(N, 16) - 10
    rope = (np.arange(N * 64).reshape(N, 64) * 5 % 256).astype(np.uint8)
    rows = ref.row400_pack(code, k, rope)
    assert rows.shape == (N, 400)
    for n in range(N):
        for e in range(512):
            nib = (rows[n, e // 2] >> (4 * (e % 2))) & 15
            sgn = (rows[n, 256 + e // 8] >> (e % 8)) & 1
            assert nib == code[n, e] & 15 and sgn == code[n, e] >> 4
        for b in range(16):
            assert np.int8(rows[n, 320 + b].view(np.int8)) == k[n, b]
        assert np.array_equal(rows[n, 336:], rope[n])
    c2, k2, r2 = ref.row400_unpack(rows)
    assert np.array_equal(c2, code) and np.array_equal(k2, k) and np.array_equal(r2, rope)


def test_row400_dequant_grid_and_e4m3_exact():
    codes = np.arange(32)[None, :].repeat(16, 0).reshape(1, 512)
    for kk in range(-12, 7):
        k = np.full((1, 16), kk)
        v = ref.row400_dequant(codes, k)[0]
        want = np.where(codes[0] & 16, -1.0, 1.0) * GRID[codes[0] & 15] * 2.0 ** kk
        assert np.array_equal(v.astype(np.float64), want)
        c = ref.row400_to_e4m3(codes, k)[0]
        dv = ref.e4m3_decode(c).astype(np.float64)
        exact = np.abs(want) >= 2.0 ** -6                # e4m3 normal range: at most 3 mantissa bits fit exactly
        assert np.array_equal(dv[exact], want[exact])
        assert np.all(np.abs(dv - want) <= 2.0 ** -10)   # below it: RNE to the 2^-9 subnormal step


def test_row400_round_trip_error():
    x = _rows(16, 3)
    code, k = ref.row400_quant(x)
    v = ref.row400_dequant(code, k).astype(np.float64)
    kk = np.repeat(k, 32, axis=1).astype(np.float64)
    y = np.abs(x.astype(np.float64)) * 2.0 ** -kk
    step = np.where(y < 2, 0.25, np.where(y < 4, 0.5, 1.0)) * 2.0 ** kk
    assert np.all(np.abs(v - x) <= step / 2 + 1e-300)


def test_row400_decode_equals_row576_write_of_the_values():
    n = 12
    g = torch.Generator().manual_seed(5)
    kv = bf16_bits(torch.randn(n, 512, generator=g) * torch.exp(torch.randn(n, 1, generator=g) * 2))
    pe = bf16_bits(torch.randn(n, 64, generator=g) * 3)
    for kv_scale in (1.0, 0.25, 3.0):
        src = np.zeros((n, 400), dtype=np.uint8)
        ref.cache_write_400(kv, pe, np.arange(n), src, kv_scale=kv_scale)
        rows = np.array([3, -1, 0, 11, 20, 5])
        g576 = ref.row400_gather(src, rows, fmt=576)
        g656 = ref.row400_gather(src, rows, fmt=656)
        code, k, rope = ref.row400_unpack(src)
        vals = ref.row400_dequant(code, k)               # exact in bf16 (at most 3 mantissa bits)
        assert np.array_equal(ref.bf16_bits_to_f32(bf16_bits(torch.from_numpy(vals))), vals)
        direct = np.zeros((n, 576), dtype=np.uint8)
        ref.cache_write_576(bf16_bits(torch.from_numpy(vals)), np.zeros((n, 64), np.uint16), np.arange(n), direct)
        for i, r in enumerate(rows):
            if 0 <= r < n:
                assert np.array_equal(g576[i, :512], direct[r, :512])
                assert np.array_equal(g576[i, 512:], src[r, 336:])
                lat6, rope6 = ref.dequant_656(g656[i:i + 1])
                lat5, rope5 = ref.dequant_576(g576[i:i + 1])
                assert np.array_equal(lat6, lat5) and np.array_equal(rope6, rope5)
            else:
                assert not g576[i].any() and not g656[i].any()


def test_e4m3_to_bf16_vs_torch():
    c = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(c).view(torch.float8_e4m3fn).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ref.e4m3_to_bf16_bits(c), want)
