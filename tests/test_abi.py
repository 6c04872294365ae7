"""CPU checks of the C-ABI library: it loads, exports every entry point include/spmla.h declares, and rejects bad
arguments with the documented codes before touching the GPU (no compute calls here)."""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    txt = open(os.path.join(ROOT, "include", "spmla.h")).read()
    return sorted(set(re.findall(r"\b(spmla_\w+)\s*\(", txt)))


def test_exports_every_declared_symbol():
    from arcagi2_flashnext_dots3_amd import _lib
    L = _lib.lib()
    declared = _declared()
    assert len(declared) >= 12
    missing = [n for n in declared if not hasattr(L, n)]
    assert not missing, missing
    assert set(declared) <= set(_lib.SIGNATURES), "ctypes signatures must cover every declared entry point"


def test_every_export_is_declared():
    """The other direction: no spmla_ entry point leaves the library without a declaration (and its citation) in
    include/spmla.h. Read from the dynamic symbol table with nm."""
    import shutil
    import subprocess
    from arcagi2_flashnext_dots3_amd import _lib
    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not available")
    out = subprocess.run([nm, "-D", "--defined-only", _lib.lib()._name], capture_output=True, text=True, check=True)
    exported = sorted({f[2] for f in (ln.split() for ln in out.stdout.splitlines())
                       if len(f) == 3 and f[1] == "T" and f[2].startswith("spmla_")})
    assert exported and sorted(set(exported) - set(_declared())) == []


def test_version():
    from arcagi2_flashnext_dots3_amd import _lib
    assert _lib.lib().spmla_version().startswith(b"spmla-gfx950")


@pytest.mark.parametrize("call,code", [
    (("spmla_attn_splitk", None, 0, 0, None, 0, None, 0, 0, None, -1, 1, 1.0, 1.0, 1, None, 0, 0, None, 0, None,
      None, None), -2),
    (("spmla_attn_splitk", None, 0, 0, None, 0, None, 0, 4096, None, 1, 1, 1.0, 1.0, 1, None, 0, 0, None, 0, None,
      None, None), -2),
    (("spmla_topk", None, 0, None, 1, 10, 5000, None, 0, 0, None), -5),
    (("spmla_topk", None, 0, None, 1, 10, 0, None, 0, 0, None), -2),
    (("spmla_topk", 256, 16, 256, 1, 10, 16, 256, 16, 2, None), -2),          # dtype 0 (fp32) or 1 (fp16) only
    (("spmla_topk_ws", None, 0, None, 1, 10, 5000, None, 0, None, 0, 0, None), -5),
    (("spmla_topk_ws", None, 0, None, 1, 10, 16, None, 0, None, 0, 1, None), -2),
    (("spmla_topk_ws_prehist", None, 0, None, 1, 10, 5000, None, 0, None, 0, 0, None), -5),
    (("spmla_topk_ws_prehist", None, 0, None, 1, 10, 0, None, 0, None, 0, 0, None), -2),
    (("spmla_index_logits_hist", None, 0, 0, None, 0, None, 0, 1, 0, None, 0, 64, None, None, 1, 64, 128, 1000, 0,
      None, 0, 0, None, 0, 0, None), -2),                                      # K = 0
    (("spmla_index_logits_hist", 256, 0, 0, 256, 0, 256, 0, 1, 0, 256, 0, 64, 256, 256, 1, 64, 128, 1000, 0,
      256, 0, 0, 8, 1 << 40, 2048, None), -2),                                 # workspace not 16-byte aligned
    # a top-k chunk of 65536 or more columns (Lc 600000): the fused histogram's 16-bit counts do not apply
    (("spmla_index_logits_hist", 256, 0, 0, 256, 0, 256, 0, 1, 0, 256, 0, 64, 256, 256, 1, 64, 128, 600000, 0,
      256, 0, 0, 256, 1 << 40, 2048, None), -5),
    (("spmla_topk_scratch", None, 0, None, 1, 10, 5000, None, 0, 0, None), -5),
    (("spmla_topk_scratch", None, 0, None, -1, 10, 16, None, 0, 1, None), -2),
    # 256 rows x 131072 columns need more workspace than the fixed 16 MiB scratch (placeholder pointers 256)
    (("spmla_topk_scratch", 256, 131072, 256, 256, 131072, 2048, 256, 2048, 0, None), -5),
    (("spmla_topk_local", None, 0, None, 1, 0, 1, 100, 4096, None, 0, None), -5),
    (("spmla_topk_local", None, 0, None, 1, 2, 2, 100, 16, None, 0, None), -2),
    (("spmla_topk_local", 256, 100, 256, 1, 0, 1, 100, 16, 256, 3, None), -2),
    (("spmla_topk_merge", None, 4, 2, 16, 33, 33, None, 0, None), -2),
    (("spmla_topk_merge", None, 4, 2, 2048, 4000, 4000, None, 0, None), -5),
    (("spmla_gather", None, 0, 650, None, 1, None, 0, None), -2),
    (("spmla_gather_pcie", None, 0, 650, None, 1, None, 0, None), -2),
    (("spmla_gather_tiers", None, 0, 656, None, 4, None, 1, 4, None, 656, None), -2),
    (("spmla_cache_write", None, 0, None, 0, None, 1, None, 10, 64, 0, 7, 1.0, None), -2),
    (("spmla_cache_write", None, 0, None, 0, None, 1, None, 10, 64, 0, 3, 1.0, None), -2),
    (("spmla_row400_gather", None, 0, None, 1, None, 656, 2, 0, None), -2),
    (("spmla_wcache_step", None, 0, 1, 8, 100, None, 10, 4, None, None, None, None, None, None, None, None, 0, 0, None,
      0, None), -2),
    (("spmla_wcache_step", None, 0, 1, 8, 1 << 32, None, 8, 4, None, None, None, None, None, None, None, None, 0, 0,
      None, 0, None), -5),
    (("spmla_wcache_step", None, 0, 1, 8, 100, None, 8, 4, None, None, None, None, None, None, None, None, 0, 2, None,
      0, None), -2),
    (("spmla_wcache_fill", None, 0, 1, 0, None, None, None, 4, None, 0, None), -2),
    (("spmla_wcache_fill", None, 0, 0, 2, None, None, None, 4, None, 0, None), -2),    # Row656 rows, Row400 lines
    (("spmla_bmm_fp8", None, 0, 0, 1, None, 0, 0, 1, None, 0, 0, 0, 0, None, 0, 0, 1, 0, 1, 1, 1, 12, None), -2),
    (("spmla_mla_query", None, 0, 0, None, 0, 0, None, None, 1, 0, None, 0, 0, None), -2),
    (("spmla_wcache_invalidate", None, 1, 10, None, 6, 4, 0, None), -2),
    (("spmla_wcache_invalidate", None, 1, 10, None, 8, 4, 3, None), -2),
    (("spmla_attn_merge", None, 0, 0, None, 0, None, 0, 0, None, 1, 1, 1.0, 1.0, None, 0, 0, None, 0, None, 0, 0,
      None, 0, None), -2),
    (("spmla_row400_gather", None, 0, None, -1, None, 656, 0, 0, None), -2),
    (("spmla_row400_copy", None, 0, None, None, 0, None, 1, 5, None), -2),
    (("spmla_row400_gather_tiers", None, 0, None, 4, None, 1, 4, None, 656, 3, None), -2),
    (("spmla_index_logits", None, 0, 0, None, 0, None, 0, 64, 0, None, 0, 64, None, None, 1, 32, 128, 10, 1, 0, 0,
      None, 0, 0, None), -5),
    (("spmla_index_logits", 256, 64, 128, 256, 64, 256, 64, 16, 2112, 256, 8, 64, 256, 256, 1, 64, 128, 64, 1, 0, 0,
      256, 64, 2, None), -2),                                               # out_dtype 0 (fp32) or 1 (fp16) only
    (("spmla_lse_merge", None, 0, 0, 0, 0, None, 0, 0, 0, 1, 1, None, 0, 0, None, None, 0, None), -2),
    # (pointer 256 below: a placeholder that the argument checks reject before anything is launched)
    (("spmla_topk_overlap", 256, 0, 0, 1, 1, 4096, 256, 256, None), -5),
    (("spmla_topk_overlap", 256, 0, 0, 0, 1, 8, 256, 256, None), -2),
    (("spmla_index_key_write_shuffle", None, 0, None, 1, None, 4, 24, 0, 0, None), -2),
    (("spmla_paged_mqa_logits", None, 0, 0, None, 0, None, 4, 64, 8448, None, 0, None, None, 1, 32, 128, 10, 0, None,
      0, None), -5),
    (("spmla_mqa_logits", 256, 8, 8, 256, 64, 256, 64, 256, 5, 256, 256, 1, 64, 128, 256, 5, None), -3),
    (("spmla_mtp_union", 256, 8, 4, 4, None, 1, 100, 8, 16, 256, 256, 256, None), -2),
    (("spmla_mtp_union", 256, 8, 4, 4, None, 1, 1 << 26, 8, 32, 256, 256, 256, None), -5),
    (("spmla_attn_packed", None, 0, 0, None, 0, None, None, None, 0, None, 4, 1, 4, 128, 3, 1.0, 1.0, 1, None, 0, 0,
      None, 0, None, None, None), -2),
    # requests of more than 6 MTP tokens are rejected, not cut to their first 6
    (("spmla_mtp_union", 256, 8, 14, 7, None, 2, 100, 8, 64, 256, 256, 256, None), -2),
    (("spmla_attn_packed", 256, 0, 0, 256, 100, 256, 256, 256, 64, None, 7, 2, 14, 128, 8, 1.0, 1.0, 1, 256, 0, 0,
      256, 0, None, None, None), -2),
    (("spmla_row576_gather", None, 0, None, -1, None, 656, None), -2),
    (("spmla_row576_gather", 256, 10, 256, 4, 256, 576, None), -3),
    # logits: local rows times P beyond 32-bit row arithmetic (R_local = INT_MAX / 4 + 1 with P = 4)
    (("spmla_index_logits", 256, 64, 128, 256, 64, 256, (2 ** 31 - 1) // 4 + 1, 16, 2112, 256, 8, 64, 256, 256, 1,
      64, 128, 64, 4, 0, 0, 256, 64, 0, None), -5),
    # Row576 attention: S > 1 needs the fp32 partials; q rows 16-byte aligned; H > 0
    (("spmla_attn576", 256, 576, 576, 256, 100, 256, 8, 8, None, 1, 1, 1.0, 1.0, 2, 256, 512, 512, 256, 1, None, None,
      None), -2),
    (("spmla_attn576", 264, 576, 576, 256, 100, 256, 8, 8, None, 1, 1, 1.0, 1.0, 1, 256, 512, 512, 256, 1, None, None,
      None), -3),
    (("spmla_attn576", 256, 576, 576, 256, 100, 256, 8, 8, None, 1, 0, 1.0, 1.0, 1, 256, 512, 512, 256, 1, None, None,
      None), -2),
    # the in-kernel split merge: a workspace is required, at most 8 splits
    (("spmla_attn", 256, 64, 64, 256, 100, 256, 8, 8, None, 1, 1, 1.0, 1.0, 4, 256, 512, 512, 256, 1, None, 0, None),
     -2),
    (("spmla_attn", 256, 64, 64, 256, 100, 256, 16, 16, None, 1, 1, 1.0, 1.0, 9, 256, 512, 512, 256, 1, 256, 1 << 30,
      None), -5),
])
def test_argument_rejection(call, code):
    from arcagi2_flashnext_dots3_amd import _lib
    assert getattr(_lib.lib(), call[0])(*call[1:]) == code


def test_attention_workspace_size():
    from arcagi2_flashnext_dots3_amd import _lib
    L = _lib.lib()
    assert L.spmla_attn_ws_bytes(64, 128, 1) == 0 and L.spmla_attn_ws_bytes(-1, 128, 4) == -1
    four = L.spmla_attn_ws_bytes(64, 128, 4)
    # the f16 partials (4 splits x 64 tokens x 128 heads x 512) plus counters, lse and exponents
    assert four >= 4 * 64 * 128 * 512 * 2 and four % 256 == 0
    assert L.spmla_attn_ws_bytes(64, 160, 4) > four                 # two head groups


def test_topk_workspace_size():
    from arcagi2_flashnext_dots3_amd import _lib
    L = _lib.lib()
    assert L.spmla_topk_ws_bytes(-1, 10, 16) == 0
    one = L.spmla_topk_ws_bytes(1, 32768, 2048)
    assert one > 0 and one % 16 == 0 and L.spmla_topk_ws_bytes(64, 32768, 2048) == 64 * one
    assert L.spmla_topk_ws_bytes(1, 131072, 2048) > one          # more chunks per row, more histograms


def test_zero_sized_calls_are_noops():
    from arcagi2_flashnext_dots3_amd import _lib
    L = _lib.lib()
    assert L.spmla_attn_splitk(None, 0, 0, None, 0, None, 0, 0, None, 0, 1, 1.0, 1.0, 1, None, 0, 0, None, 0,
                               None, None, None) == 0
    assert L.spmla_topk(None, 0, None, 0, 10, 16, None, 0, 0, None) == 0
    assert L.spmla_gather(None, 0, 656 - 656 % 16, None, 0, None, 0, None) == 0


def test_product_package_does_not_import_oracle():
    pkg = os.path.join(ROOT, "arcagi2_flashnext_dots3_amd")
    for dp, _, fs in os.walk(pkg):
        for f in fs:
            if f.endswith(".py"):
                txt = open(os.path.join(dp, f)).read()
                assert "oracle" not in re.findall(r"^\s*(?:from|import)\s+(\w+)", txt, re.M), f


@pytest.mark.parametrize("lang", ["c", "c++"])
def test_header_compiles_standalone(tmp_path, lang):
    """include/spmla.h is a plain C-ABI header: it compiles on its own as C99 and as C++17 with warnings as errors."""
    import shutil
    import subprocess
    cc = shutil.which("gcc" if lang == "c" else "g++")
    if cc is None:
        pytest.skip("no host compiler")
    src = tmp_path / "hdr.c"
    src.write_text('#include "spmla.h"\nint main(void) { return 0; }\n')
    std = "-std=c99" if lang == "c" else "-std=c++17"
    r = subprocess.run([cc, std, "-Wall", "-Werror", "-fsyntax-only", "-I", os.path.join(ROOT, "include"), "-x", lang,
                        str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
