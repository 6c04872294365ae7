"""Exact top-k for the DSA indexer: the reference's fast_topk module (dotsnote/engine/arcstats_pkg/arcstats/
fast_topk.py:1-78) on libspmla_gfx950.so.

local(lg, ctx, rank, P, kl)        -> [rows, 2 kl] payload [top-kl values | positions], ascending column order
merge(allp, n, P, kl, kk, out)     -> out [n, topk_tokens] int32 positions sorted by (value desc, index asc)
Selection is torch.topk's: order-preserving key (-0 < +0, NaN largest), equal values -> lower column. Unlike the
reference there is no torch fallback: the library is required (a missing library raises).
"""
from . import _lib, kernels

MODE = "2"   # both stages always run on the library


def lib():
    return _lib.lib()


def enabled(level=1):
    return True


def local(lg, ctx, rank, P, kl, pk=None, nt=None, agg=None):
    """lg [rows, Lc] fp32 or fp16 (column j = position j * P + rank; columns at or beyond the row's ctx are never read),
    ctx int32 [rows] -> pk [rows, 2 * kl] fp32 = [top-kl values | their positions (int32 bits)], selected columns in
    ascending column order; rows with fewer than kl valid columns padded with -inf (fast_topk.py:52-66).
    nt / agg (the reference's CTA-size knobs) are accepted and ignored."""
    return kernels.topk_local(lg, ctx, rank, P, kl, pk)


def merge(allp, n, P, kl, kk, out, nt=None):
    """allp [P * n, 2 * kl] all-gathered payloads (rank-major) -> out [n, topk_tokens] int32: positions of the top kk
    (value desc, concatenation index asc), -1 where the value is +-inf and for columns >= kk (fast_topk.py:69-78)."""
    return kernels.topk_merge(allp, n, P, kl, kk, out)
