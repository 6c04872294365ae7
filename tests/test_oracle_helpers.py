"""Pins of the oracle's small helpers against library routines and their defining properties: bf16 conversions
against torch's, the top-k order key against numpy's float order, and the Row656 / Row576 decoders against torch's
float8_e4m3fn decode with the scales and rope bytes placed by hand. CPU only."""
import numpy as np
import torch

from oracle import spmla_ref as ref


def _f32_cases(n=1 << 16):
    g = np.random.default_rng(0)
    x = g.standard_normal(n).astype(np.float32) * np.exp2(g.integers(-140, 120, n)).astype(np.float32)
    # exact ties at bf16 precision (low 16 bits 0x8000), both parities, and the specials
    t = (g.integers(0, 1 << 16, 4096).astype(np.uint32) << 16) | 0x8000
    sp = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 3.4028235e38, -3.4028235e38,
                   1.1754944e-38], dtype=np.float32)
    return np.concatenate([x, t.view(np.float32), sp])


def test_bf16_conversions_match_torch():
    x = _f32_cases()
    got = ref.f32_to_bf16_bits(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all(np.isnan(ref.bf16_bits_to_f32(got[nan])))       # NaN stays NaN (quiet)
    back = ref.bf16_bits_to_f32(want[~nan])
    assert np.array_equal(back.view(np.uint32),
                          torch.from_numpy(want[~nan].view(np.int16)).view(torch.bfloat16).float().numpy()
                          .view(np.uint32))


def test_okey_orders_like_floats():
    x = _f32_cases(1 << 14)
    fin = x[~np.isnan(x)]
    k = ref.okey(fin)
    order = np.argsort(k, kind="stable")
    s = fin[order]
    assert np.all(s[:-1] <= s[1:])                                  # keys sort the values ascending
    assert ref.okey(np.float32(-0.0)) < ref.okey(np.float32(0.0))   # -0 below +0
    assert ref.okey(np.float32(np.nan)) == 0xFFFFFFFF and ref.okey(np.float32(np.inf)) < 0xFFFFFFFF


def test_dequant_656_and_576_match_torch_float8():
    g = np.random.default_rng(1)
    n = 64
    rows = g.integers(0, 256, (n, 656), dtype=np.uint8)
    rows[:, :512][(rows[:, :512] & 0x7F) == 0x7F] = 0x10          # no NaN codes
    sc = (g.random((n, 4)) * 3 + 0.01).astype(np.float32)
    rows[:, 512:528] = sc.view(np.uint8).reshape(n, 16)
    rope = ref.f32_to_bf16_bits(g.standard_normal((n, 64)).astype(np.float32))
    rows[:, 528:656] = rope.view(np.uint8).reshape(n, 128)
    lat, rp = ref.dequant_656(rows)
    codes = torch.from_numpy(rows[:, :512].copy()).view(torch.float8_e4m3fn).double().view(n, 4, 128)
    want = (codes * torch.from_numpy(sc).double()[:, :, None]).view(n, 512).numpy()
    assert np.array_equal(lat, want)
    assert np.array_equal(rp, torch.from_numpy(rope.view(np.int16)).view(torch.bfloat16).double().numpy())
    r576 = rows[:, :576].copy()
    r576[:, 512:][(r576[:, 512:] & 0x7F) == 0x7F] = 0x10
    a, b = ref.dequant_576(r576)
    v = torch.from_numpy(r576).view(torch.float8_e4m3fn).double().numpy()
    assert np.array_equal(a, v[:, :512]) and np.array_equal(b, v[:, 512:])


def test_every_oracle_function_names_its_pin():
    """Each public function of the oracle has an entry in PINS saying what checks it."""
    import ast
    import os
    src = open(os.path.join(os.path.dirname(ref.__file__), "spmla_ref.py")).read()
    fns = [n.name for n in ast.parse(src).body if isinstance(n, ast.FunctionDef) and not n.name.startswith("_")]
    assert [f for f in fns if f not in ref.PINS] == []
