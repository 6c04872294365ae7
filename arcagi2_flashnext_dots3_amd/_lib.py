"""ctypes binding of libspmla_gfx950.so (the C-ABI declared in include/spmla.h).

Mirrors the reference's loaders (dotsnote/engine/arcstats_pkg/arcstats/offload_cuda2.py:21-47,
fast_topk.py:29-45): CDLL of an env override or the library next to this file, argtypes per entry point, and an int
return code turned into RuntimeError. Unlike the reference there is no silent fallback: a missing library raises.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("SPMLA_LIB") or os.path.join(_HERE, "libspmla_gfx950.so")

P = ctypes.c_void_p
LL = ctypes.c_longlong
I = ctypes.c_int
F = ctypes.c_float

# name -> argtypes (all return int unless listed in _RESTYPE)
SIGNATURES = {
    "spmla_cache_write": [P, LL, P, LL, P, I, P, LL, I, LL, I, F, P],
    "spmla_index_key_write": [P, LL, P, I, P, LL, I, I, I, LL, I, P],
    "spmla_index_logits": [P, LL, LL, P, LL, P, LL, I, LL, P, LL, I, P, P, I, I, I, I, I, I, I, P, LL, I, P],
    "spmla_topk": [P, LL, P, I, I, I, P, LL, I, P],
    "spmla_topk_ws_bytes": [I, I, I],
    "spmla_topk_ws": [P, LL, P, I, I, I, P, LL, P, LL, I, P],
    "spmla_topk_ws_prehist": [P, LL, P, I, I, I, P, LL, P, LL, I, P],
    "spmla_index_logits_hist": [P, LL, LL, P, LL, P, LL, I, LL, P, LL, I, P, P, I, I, I, I, I, P, LL, I, P, LL, I, P],
    "spmla_topk_scratch_bytes": [],
    "spmla_topk_scratch": [P, LL, P, I, I, I, P, LL, I, P],
    "spmla_topk_local": [P, LL, P, I, I, I, I, I, P, I, P],
    "spmla_topk_merge": [P, I, I, I, I, I, P, LL, P],
    "spmla_rows_from_topk": [P, LL, P, P, LL, I, I, LL, I, I, P, LL, P, P],
    "spmla_gather": [P, LL, I, P, I, P, LL, P],
    "spmla_gather_pcie": [P, LL, I, P, I, P, LL, P],
    "spmla_gather_tiers": [P, LL, I, P, LL, P, I, I, P, LL, P],
    "spmla_copy_rows": [P, LL, P, P, LL, P, I, I, P],
    "spmla_row400_gather": [P, LL, P, I, P, LL, I, I, P],
    "spmla_row576_gather": [P, LL, P, I, P, LL, P],
    "spmla_row400_copy": [P, LL, P, P, LL, P, I, I, P],
    "spmla_row400_gather_tiers": [P, LL, P, LL, P, I, I, P, LL, I, P],
    "spmla_row400_decode_tiers": [P, LL, P, LL, P, I, I, P, LL, I, P],
    "spmla_tier_split": [P, LL, I, I, P, LL, P, LL, P, P, LL, P, P],
    "spmla_wcache_step": [P, LL, I, I, LL, P, I, I, P, P, P, P, P, P, P, P, I, I, P, LL, P],
    "spmla_wcache_place": [P, LL, I, I, LL, P, I, I, P, P, P, P, P, P, P, P, I, I, P],
    "spmla_wcache_resolve": [P, LL, I, I, LL, P, I, I, P, P, P, P, P, P, P, P, I, I, P, LL, P],
    "spmla_wcache_fill": [P, LL, I, I, P, P, P, I, P, LL, P],
    "spmla_wcache_invalidate": [P, I, LL, P, I, I, I, P],
    "spmla_split_res": [P, LL, P, LL, I, I, P, LL, P, P, LL, P, P],
    "spmla_wcache_split": [P, LL, I, I, P, I, P, P, LL, P, P, LL, P, P],
    "spmla_compact_stage": [P, I, P, LL, I, I, P, P, P, P, LL, P],
    "spmla_attn_splitk": [P, LL, LL, P, LL, P, LL, I, P, I, I, F, F, I, P, LL, LL, P, LL, P, P, P],
    "spmla_attn576": [P, LL, LL, P, LL, P, LL, I, P, I, I, F, F, I, P, LL, LL, P, LL, P, P, P],
    "spmla_attn": [P, LL, LL, P, LL, P, LL, I, P, I, I, F, F, I, P, LL, LL, P, LL, P, LL, P],
    "spmla_attn_ws_bytes": [I, I, I],
    "spmla_attn_merge": [P, LL, LL, P, LL, P, LL, I, P, I, I, F, F, P, LL, LL, P, LL, P, LL, LL, P, LL, P],
    "spmla_lse_merge": [P, I, LL, LL, LL, P, LL, LL, I, I, I, P, LL, LL, P, P, LL, P],
    "spmla_bmm_fp8": [P, LL, LL, LL, P, LL, LL, LL, P, LL, LL, LL, I, P, LL, LL, LL, I, I, I, I, I, P],
    "spmla_mla_query": [P, LL, LL, P, LL, LL, P, P, I, I, P, LL, LL, P],
    "spmla_topk_overlap": [P, LL, LL, I, I, I, P, P, P],
    "spmla_mtp_union": [P, LL, I, I, P, I, LL, I, I, P, P, P, P],
    "spmla_attn_packed": [P, LL, LL, P, LL, P, P, P, I, P, I, I, I, I, I, F, F, I, P, LL, LL, P, LL, P, P, P],
    "spmla_index_key_write_shuffle": [P, LL, P, I, P, LL, I, LL, I, P],
    "spmla_mqa_logits": [P, LL, LL, P, LL, P, LL, P, I, P, P, I, I, I, P, LL, P],
    "spmla_paged_mqa_logits": [P, LL, LL, P, LL, P, LL, I, LL, P, LL, P, P, I, I, I, I, I, P, LL, P],
    "spmla_version": [],
    "spmla_host_e4m3_encode": [P, P, LL],
}
_RESTYPE = {"spmla_version": ctypes.c_char_p, "spmla_host_e4m3_encode": None, "spmla_topk_ws_bytes": LL,
            "spmla_topk_scratch_bytes": LL, "spmla_attn_ws_bytes": LL}

ERRORS = {-2: "bad argument", -3: "misaligned pointer or stride", -5: "size beyond the kernel's limit"}

_L = None


def lib():
    """The loaded library; raises if it is missing (build it with arcagi2_flashnext_dots3_amd.build)."""
    global _L
    if _L is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} not found: build it (python -m arcagi2_flashnext_dots3_amd.build)")
        L = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = _RESTYPE.get(name, ctypes.c_int)
        _L = L
    return _L


def call(name, *args):
    """Invoke entry point `name`; a nonzero return code raises RuntimeError naming the entry point."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        raise RuntimeError(f"{name} failed: {rc} ({ERRORS.get(rc, 'hip error')})")
    return rc


def exported_symbols():
    return [n for n in SIGNATURES if hasattr(lib(), n)]
