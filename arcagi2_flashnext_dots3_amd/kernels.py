"""Tensor-level wrappers of the C-ABI entry points (include/spmla.h): argument checks, strides, the caller's stream.

Each wrapper mirrors the Python side of the reference kernel it replaces (offload_cuda2.attend,
offload_cuda.split_partials, fast_topk.local/merge, ShardStore.write/logits, LayerOffload.gather), raises
RuntimeError on a failed launch and never falls back to a CPU path.
"""
import torch

from . import _lib

D_LAT, D_ROPE, D_QK = 512, 64, 576
ROW656, ROW576, ROW400, KEYROW = 656, 576, 400, 132
_ROWB = {0: ROW656, 1: ROW576, 2: ROW400}        # cache_write formats
LOG2E = 1.4426950408889634


def _stream(t):
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t):
    return t.data_ptr() if t is not None else None


def _need(cond, msg):
    if not cond:
        raise ValueError(msg)


# ---------------------------------------------------------------------------------------------- cache write
def cache_write(kv_c, k_pe, slots, cache, fmt=0, kv_scale=1.0, block_size=None, block_stride=None):
    """kv_c [n, 512] bf16, k_pe [n, 64] or [n, 1, 64] bf16, slots [n] int64 -> rows of `cache` (uint8, Row656
    (fmt 0), Row576 (fmt 1) or Row400 (fmt 2, the compact e2m2b32 row)). cache is [R, row] or paged
    [blocks, block_size, row] (block stride may be padded)."""
    kpe = k_pe.reshape(k_pe.shape[0], -1)
    n = min(kv_c.shape[0], slots.shape[0])
    _need(fmt in _ROWB, f"fmt must be one of {sorted(_ROWB)}")
    rowb = _ROWB[fmt]
    _need(kv_c.dtype == torch.bfloat16 and kpe.dtype == torch.bfloat16, "kv_c / k_pe must be bf16")
    _need(kv_c.shape[1] == D_LAT and kpe.shape[1] == D_ROPE and kv_c.stride(1) == 1 and kpe.stride(1) == 1,
          "kv_c [n, 512] / k_pe [n, 64] with contiguous rows")
    _need(cache.dtype == torch.uint8 and cache.shape[-1] == rowb and cache.stride(-1) == 1, "cache rows of uint8")
    _need(slots.dtype == torch.int64, "slots int64")
    if cache.dim() == 3:
        bs, bstride, R = cache.shape[1], cache.stride(0), cache.shape[0] * cache.shape[1]
        _need(cache.stride(1) == rowb, "rows inside a block must be contiguous")
    else:
        R = cache.shape[0]
        bs = block_size or max(1, R)
        bstride = block_stride or bs * rowb
    _lib.call("spmla_cache_write", kv_c.data_ptr(), kv_c.stride(0), kpe.data_ptr(), kpe.stride(0), slots.data_ptr(),
              n, cache.data_ptr(), R, bs, bstride, int(fmt), float(kv_scale), _stream(kv_c))


def index_key_write(k, slots, store, P=1, rank=0, ue8m0=False):
    """k [n, 128] bf16 -> store [blocks, rows_per_block, 132] (or [R, 132]) uint8 rows of this rank."""
    n = min(k.shape[0], slots.shape[0])
    _need(k.dtype == torch.bfloat16 and k.shape[1] == 128 and k.stride(1) == 1, "k [n, 128] bf16")
    _need(store.dtype == torch.uint8 and store.shape[-1] == KEYROW, "store rows of 132 bytes")
    if store.dim() == 3:
        rpb, bstride, R = store.shape[1], store.stride(0), store.shape[0] * store.shape[1]
    else:
        R = store.shape[0]
        rpb, bstride = max(1, R), max(1, R) * KEYROW
    _lib.call("spmla_index_key_write", k.data_ptr(), k.stride(0), slots.data_ptr(), n, store.data_ptr(), R, P, rank,
              rpb, bstride, int(bool(ue8m0)), _stream(k))


def _shuffle_cache(kv_cache):
    """vLLM's indexer key cache [blocks, bs, 1, 132] / [blocks, bs, 132] / [blocks, bs * 132] uint8 -> (blocks, bs,
    block stride in bytes)."""
    _need(kv_cache.dtype == torch.uint8, "indexer key cache must be uint8")
    if kv_cache.dim() >= 3:
        nb, bs = kv_cache.shape[0], kv_cache.shape[1]
        _need(kv_cache[0].numel() == bs * KEYROW, "indexer key cache rows of 132 bytes")
    else:
        nb, bs = kv_cache.shape[0], kv_cache.shape[1] // KEYROW
    _need(bs % 16 == 0, "SHUFFLE layout needs a block size that is a multiple of 16")
    return nb, bs, kv_cache.stride(0)


def index_key_write_shuffle(k, slots, kv_cache, ue8m0=False):
    """k [n, 128] bf16 -> vLLM's paged indexer key cache in the SHUFFLE layout (dsa_sm89.py:63-66): the same
    per-key quantization as index_key_write, slot = block * bs + offset."""
    n = min(k.shape[0], slots.shape[0])
    _need(k.dtype == torch.bfloat16 and k.shape[1] == 128 and k.stride(1) == 1, "k [n, 128] bf16")
    nb, bs, bstride = _shuffle_cache(kv_cache)
    _lib.call("spmla_index_key_write_shuffle", k.data_ptr(), k.stride(0), slots.data_ptr(), n, kv_cache.data_ptr(),
              nb, bs, bstride, int(bool(ue8m0)), _stream(k))


def paged_ctx(seq_lens, next_n):
    """Per logits row b * next_n + j: (request b, visible keys): seq_lens[b] - (next_n - 1 - j), or seq_lens[b, j]
    for 2-D seq_lens (dsa_sm89.py:46-53). int32 tensors on seq_lens' device."""
    B = seq_lens.shape[0]
    dev = seq_lens.device
    req = torch.arange(B * next_n, device=dev, dtype=torch.int32) // next_n
    if seq_lens.dim() == 2:
        ctx = seq_lens.reshape(-1).to(torch.int32)
    else:
        j = torch.arange(next_n, device=dev, dtype=torch.int32).repeat(B)
        ctx = (seq_lens.to(torch.int32)[req.long()] - (next_n - 1 - j)).to(torch.int32)
    return req.contiguous(), ctx.contiguous()


def paged_mqa_logits(q, kv_cache, weights, seq_lens, block_table, max_model_len, out=None):
    """paged_mqa_logits_triton (dsa_sm89.py:75-94): q [B, next_n, 64, 128] (bf16, or float8_e4m3fn widened exactly
    to bf16), kv_cache vLLM's SHUFFLE indexer cache, weights [B * next_n, 64] fp32, seq_lens [B] or [B, next_n],
    block_table [B, cols] int32 -> logits [B * next_n, max_model_len] fp32, -inf outside each row's context."""
    B, nn, H, D = q.shape
    if q.dtype == torch.float8_e4m3fn:
        q = q.to(torch.bfloat16)
    _need(q.dtype == torch.bfloat16 and q.stride(3) == 1, "q bf16 / e4m3 with contiguous head dim")
    qr = q.reshape(B * nn, H, D)
    _need(weights.dtype == torch.float32 and weights.stride(1) == 1, "weights fp32")
    _need(block_table.dtype == torch.int32, "int32 block table")
    nb, bs, bstride = _shuffle_cache(kv_cache)
    req, ctx = paged_ctx(seq_lens, nn)
    rows = B * nn
    if out is None:
        out = torch.empty(rows, max(max_model_len, 1), dtype=torch.float32, device=q.device)
    _lib.call("spmla_paged_mqa_logits", qr.data_ptr(), qr.stride(0), qr.stride(1), weights.data_ptr(),
              weights.stride(0), kv_cache.data_ptr(), nb, bs, bstride, block_table.data_ptr(), block_table.stride(0),
              req.data_ptr(), ctx.data_ptr(), rows, H, D, max_model_len, 0, out.data_ptr(), out.stride(0), _stream(q))
    return out


def mqa_logits(q, kv, weights, cu_seqlen_ks, cu_seqlen_ke):
    """mqa_logits_triton (dsa_sm89.py:121-133), the prefill logits over gathered keys: q [M, 64, 128] (bf16, or
    float8_e4m3fn widened exactly), kv = (codes [N, 128] e4m3 / uint8, scales [N] or [N, 1] fp32), weights [M, 64]
    fp32, key range [ks[m], ke[m]) per row (int32) -> [M, N] fp32, -inf outside the range."""
    codes, scales = kv
    M, H, D = q.shape
    N = codes.shape[0]
    if q.dtype == torch.float8_e4m3fn:
        q = q.to(torch.bfloat16)
    _need(q.dtype == torch.bfloat16 and q.stride(2) == 1, "q bf16 / e4m3 with contiguous head dim")
    codes = codes.view(torch.uint8) if codes.dtype != torch.uint8 else codes
    _need(codes.dim() == 2 and codes.shape[1] == 128 and codes.stride(1) == 1, "codes [N, 128]")
    sc = scales.reshape(-1).contiguous()
    _need(sc.dtype == torch.float32 and sc.numel() == N, "scales [N] fp32")
    ks = cu_seqlen_ks.to(torch.int32).contiguous()
    ke = cu_seqlen_ke.to(torch.int32).contiguous()
    out = torch.empty(M, N, dtype=torch.float32, device=q.device)
    _lib.call("spmla_mqa_logits", q.data_ptr(), q.stride(0), q.stride(1), weights.data_ptr(), weights.stride(0),
              codes.data_ptr(), codes.stride(0), sc.data_ptr(), N, ks.data_ptr(), ke.data_ptr(), M, H, D,
              out.data_ptr(), out.stride(0), _stream(q))
    return out


# ---------------------------------------------------------------------------------------------- indexer
# logits element types of the indexer kernels: the C-ABI's dtype argument
_LG_DT = {torch.float32: 0, torch.float16: 1}


def index_logits(q, w, store, block_table, block_size, req, ctx, Lc, out=None, P=1, rank=0, noinf=False,
                 dtype=torch.float32):
    """q [rows, 64, 128] bf16, w [rows, 64] fp32, store [blocks, rpb, 132] uint8, block_table [nreq, cols] int32,
    req / ctx [rows] int32 -> logits [rows, Lc] (column j = position j * P + rank) in fp32, or in fp16 with
    dtype=torch.float16 (each fp32 logit rounded to nearest even: the reference's ARC_SHARD_F16OUT)."""
    rows, H, D = q.shape
    _need(q.dtype == torch.bfloat16 and q.stride(2) == 1, "q bf16 with contiguous head dim")
    _need(w.dtype == torch.float32 and w.stride(1) == 1, "w fp32")
    _need(req.dtype == torch.int32 and ctx.dtype == torch.int32 and block_table.dtype == torch.int32, "int32 tables")
    if store.dim() == 3:
        rpb, bstride, R = store.shape[1], store.stride(0), store.shape[0] * store.shape[1]
    else:
        R = store.shape[0]
        rpb, bstride = max(1, R), max(1, R) * KEYROW
    if out is None:
        out = torch.empty(rows, max(Lc, 1), dtype=dtype, device=q.device)
    _need(out.dtype in _LG_DT and out.stride(1) == 1 and out.shape[0] >= rows and out.shape[1] >= Lc,
          "out fp32 / fp16 [rows, >= Lc] with contiguous rows")
    _lib.call("spmla_index_logits", q.data_ptr(), q.stride(0), q.stride(1), w.data_ptr(), w.stride(0),
              store.data_ptr(), R, rpb, bstride, block_table.data_ptr(), block_table.stride(0), block_size,
              req.data_ptr(), ctx.data_ptr(), rows, H, D, Lc, P, rank, int(bool(noinf)), out.data_ptr(),
              out.stride(0), _LG_DT[out.dtype], _stream(q))
    return out


_WS = {}
_WS_CNT = {}      # attention workspaces: counter bytes of the last launch (the bytes known to be zero)
_WS_KEEP = []     # every workspace ever handed out: a HIP graph captured with one keeps its address for good


def _workspace(kind, device, nbytes, zero=False):
    """Device workspace of one kind of call, per (device, current stream): calls queued on one stream run in order,
    so they can share it; calls on other streams get their own. Grown on demand (at least doubling); a replaced
    buffer stays allocated, so graphs captured with it stay valid. zero: allocated zero-filled (the attention's
    counters). Under HIP graph capture nothing is allocated (a buffer allocated there would hold its contents only
    after the first replay): the device's largest workspace of this kind from an eager call serves every capture, so
    graphs that use it must be replayed one at a time, and a capture needing more raises. Returns (buffer, key);
    key is None under capture."""
    dev = torch.device(device)
    if torch.cuda.is_current_stream_capturing():
        have = [b for (k, d, _), b in _WS.items() if k == kind and d == dev]
        b = max(have, key=lambda t: t.numel(), default=None)
        _need(b is not None and b.numel() >= nbytes,
              f"{kind} workspace of {nbytes} bytes needed under HIP graph capture: pass one explicitly, or make an "
              f"eager call of at least this size (reserve_workspace) before capturing")
        return b, None
    key = (kind, dev, torch.cuda.current_stream(dev).cuda_stream)
    b = _WS.get(key)
    if b is None or b.numel() < nbytes:
        n = max(nbytes, 256, 2 * b.numel() if b is not None else 0)
        b = torch.zeros(n, dtype=torch.uint8, device=dev) if zero else torch.empty(n, dtype=torch.uint8, device=dev)
        _WS[key] = b
        _WS_KEEP.append(b)
        _WS_CNT[key] = n if zero else 0
    return b, key


def fused_max_tokens(H, cus=256):
    """The most tokens for which auto_split picks the in-kernel split merge (H heads): below it attend needs a
    workspace."""
    return max(0, -(-cus * 3 // (8 * ((H + 31) // 32))) - 1)


def reserve_workspace(device, H, T=None, split=8):
    """Allocate now (eagerly) the attention workspace that attend's split merge needs for up to T tokens of H heads
    (default: every size auto_split sends there), so that later HIP graph captures find it. No-op when present."""
    T = fused_max_tokens(H) if T is None else T
    if T > 0:
        _workspace("attn", device, int(_lib.lib().spmla_attn_ws_bytes(T, H, split)), zero=True)


def _attn_counter_bytes(T, H):
    """Leading counter bytes of spmla_attn's workspace: 4 per (token, group of 128 heads), 256-byte rounded."""
    return (4 * T * ((H + 127) // 128) + 255) // 256 * 256


def topk(logits, ctx, K, out=None, single_pass=False, ws=None):
    """logits [rows, Lc] fp32 or fp16, ctx [rows] int32 -> [rows, K] int32 positions (value desc, position asc; -1
    pad). Several workgroups per row (spmla_topk_ws; ws: a uint8 workspace, else a cached one of
    spmla_topk_ws_bytes) unless single_pass (spmla_topk, one workgroup per row)."""
    rows, Lc = logits.shape
    _need(logits.dtype in _LG_DT and logits.stride(1) == 1, "fp32 / fp16 logits with contiguous rows")
    _need(ctx.dtype == torch.int32 and ctx.is_contiguous(), "ctx int32")
    if out is None:
        out = torch.empty(rows, K, dtype=torch.int32, device=logits.device)
    _need(out.dtype == torch.int32 and out.stride(1) == 1 and out.shape[0] >= rows and out.shape[1] >= K,
          "out int32 [rows, >= K] with contiguous rows")
    if single_pass:
        _lib.call("spmla_topk", logits.data_ptr(), logits.stride(0), ctx.data_ptr(), rows, Lc, K, out.data_ptr(),
                  out.stride(0), _LG_DT[logits.dtype], _stream(logits))
        return out
    nb = int(_lib.lib().spmla_topk_ws_bytes(rows, Lc, K))
    if ws is None:
        ws, _ = _workspace("topk", logits.device, nb)
    _lib.call("spmla_topk_ws", logits.data_ptr(), logits.stride(0), ctx.data_ptr(), rows, Lc, K, out.data_ptr(),
              out.stride(0), ws.data_ptr(), ws.numel(), _LG_DT[logits.dtype], _stream(logits))
    return out



def topk_prehist(logits, ctx, K, ws, out=None):
    """topk over logits whose first-level histograms spmla_index_logits_hist already wrote into ws (same rows, Lc, K,
    ctx and dtype; spmla_topk_ws_prehist): the histogram pass is skipped, the result is topk's."""
    rows, Lc = logits.shape
    _need(logits.dtype in _LG_DT and logits.stride(1) == 1, "fp32 / fp16 logits with contiguous rows")
    _need(ctx.dtype == torch.int32 and ctx.is_contiguous(), "ctx int32")
    if out is None:
        out = torch.empty(rows, K, dtype=torch.int32, device=logits.device)
    _need(out.dtype == torch.int32 and out.stride(1) == 1 and out.shape[0] >= rows and out.shape[1] >= K,
          "out int32 [rows, >= K] with contiguous rows")
    _lib.call("spmla_topk_ws_prehist", logits.data_ptr(), logits.stride(0), ctx.data_ptr(), rows, Lc, K,
              out.data_ptr(), out.stride(0), ws.data_ptr(), ws.numel(), _LG_DT[logits.dtype], _stream(logits))
    return out


def logits_hist(q, w, base, R, rpb, bstride, block_table, block_size, req, ctx, Lc, K, lg, ws, noinf=False):
    """spmla_index_logits_hist (P = 1): the logits into lg [rows, >= Lc] (fp32 / fp16) and the first-level top-k
    histograms into ws. Returns False without a launch when the fused path does not apply (a top-k chunk of 65536 or
    more columns); the caller then runs the logits and topk separately."""
    rows = q.shape[0]
    rc = _lib.lib().spmla_index_logits_hist(
        q.data_ptr(), q.stride(0), q.stride(1), w.data_ptr(), w.stride(0), base.data_ptr(), R, rpb, bstride,
        block_table.data_ptr(), block_table.stride(0), block_size, req.data_ptr(), ctx.data_ptr(), rows, q.shape[1],
        q.shape[2], Lc, int(bool(noinf)), lg.data_ptr(), lg.stride(0), _LG_DT[lg.dtype], ws.data_ptr(), ws.numel(),
        K, _stream(q))
    if rc == -5:
        return False
    if rc != 0:
        raise RuntimeError(f"spmla_index_logits_hist failed: {rc} ({_lib.ERRORS.get(rc, 'hip error')})")
    return True


def logits_topk(q, w, store, block_table, block_size, req, ctx, Lc, K, lg=None, out=None, noinf=False,
                dtype=torch.float32, ws=None):
    """index_logits (P = 1) then topk of its [rows, Lc] logits, with the top-k's first histogram pass done in the
    logits epilogue (logits_hist + topk_prehist) when it applies, else the two separate calls; same logits and
    positions either way. Returns (logits, positions)."""
    rows, H, D = q.shape
    _need(q.dtype == torch.bfloat16 and q.stride(2) == 1, "q bf16 with contiguous head dim")
    _need(w.dtype == torch.float32 and w.stride(1) == 1, "w fp32")
    _need(req.dtype == torch.int32 and ctx.dtype == torch.int32 and block_table.dtype == torch.int32, "int32 tables")
    _need(ctx.is_contiguous(), "ctx int32 contiguous")
    if store.dim() == 3:
        rpb, bstride, R = store.shape[1], store.stride(0), store.shape[0] * store.shape[1]
    else:
        R = store.shape[0]
        rpb, bstride = max(1, R), max(1, R) * KEYROW
    if lg is None:
        lg = torch.empty(rows, max(Lc, 1), dtype=dtype, device=q.device)
    _need(lg.dtype in _LG_DT and lg.stride(1) == 1 and lg.shape[0] >= rows and lg.shape[1] >= Lc,
          "logits fp32 / fp16 [rows, >= Lc] with contiguous rows")
    if out is None:
        out = torch.empty(rows, K, dtype=torch.int32, device=q.device)
    if rows == 0 or Lc == 0:
        out[:rows, :K] = -1
        return lg, out
    lgv = lg[:rows, :Lc]
    if ws is None:
        ws, _ = _workspace("topk", q.device, int(_lib.lib().spmla_topk_ws_bytes(rows, Lc, K)))
    if logits_hist(q, w, store, R, rpb, bstride, block_table, block_size, req, ctx, Lc, K, lg, ws, noinf):
        topk_prehist(lgv, ctx, K, ws, out=out)
    else:
        index_logits(q, w, store, block_table, block_size, req, ctx, Lc, out=lg, noinf=noinf)
        topk(lgv, ctx, K, out=out, ws=ws)
    return lg, out

def topk_scratch(logits, ctx, K, out=None):
    """topk without a workspace or any allocation in the library (spmla_topk_scratch): the passes use the library's
    fixed per-GPU scratch. Calls that overlap on one GPU race. Sizes beyond the scratch raise (SPMLA_ELIMIT)."""
    rows, Lc = logits.shape
    _need(logits.dtype in _LG_DT and logits.stride(1) == 1, "fp32 / fp16 logits with contiguous rows")
    _need(ctx.dtype == torch.int32 and ctx.is_contiguous() and ctx.shape[0] >= rows, "ctx int32 [rows]")
    if out is None:
        out = torch.empty(rows, K, dtype=torch.int32, device=logits.device)
    _need(out.dtype == torch.int32 and out.stride(1) == 1 and out.shape[0] >= rows and out.shape[1] >= K,
          "out int32 [rows, >= K]")
    _lib.call("spmla_topk_scratch", logits.data_ptr(), logits.stride(0), ctx.data_ptr(), rows, Lc, K,
              out.data_ptr(), out.stride(0), _LG_DT[logits.dtype], _stream(logits))
    return out


def topk_local(lg, ctx, rank, P, kl, pk=None):
    """fast_topk.local: lg [rows, Lc] fp32 or fp16 (column j = position j * P + rank), ctx [rows] int32 positions ->
    pk [rows, 2 * kl] fp32 = [top-kl values | their positions as int32 bits], ascending column order, -inf padded."""
    rows, Lc = lg.shape
    _need(lg.dtype in _LG_DT and lg.stride(1) == 1, "fp32 / fp16 logits with contiguous rows")
    _need(ctx.dtype == torch.int32 and ctx.is_contiguous(), "ctx int32")
    if pk is None:
        pk = torch.empty(rows, 2 * kl, dtype=torch.float32, device=lg.device)
    _need(pk.dtype == torch.float32 and pk.is_contiguous() and pk.shape[-1] == 2 * kl, "pk [rows, 2 * kl] fp32")
    _lib.call("spmla_topk_local", lg.data_ptr(), lg.stride(0), ctx.data_ptr(), rows, rank, P, Lc, kl, pk.data_ptr(),
              _LG_DT[lg.dtype], _stream(lg))
    return pk


def topk_merge(allp, n, P, kl, kk, out):
    """fast_topk.merge: allp [P * n, 2 * kl] rank-major payloads -> out [n, topk_tokens] int32 positions."""
    _need(allp.dtype == torch.float32 and allp.is_contiguous(), "allp fp32 contiguous")
    _need(out.dtype == torch.int32 and out.stride(1) == 1, "out int32 with contiguous rows")
    _lib.call("spmla_topk_merge", allp.data_ptr(), n, P, kl, kk, out.shape[1], out.data_ptr(), out.stride(0),
              _stream(allp))
    return out


def rows_from_topk(topk_pos, req, block_table, block_size, stride_rows=None, rows=None, counts=None):
    """Request-local positions [T, K] -> global rows [T, K] int32 (vLLM triton_convert_req_index_to_global_index)."""
    T, K = topk_pos.shape
    if rows is None:
        rows = torch.empty(T, K, dtype=torch.int32, device=topk_pos.device)
    _lib.call("spmla_rows_from_topk", topk_pos.data_ptr(), topk_pos.stride(0), req.data_ptr(),
              block_table.data_ptr(), block_table.stride(0), block_table.shape[1], block_size,
              stride_rows if stride_rows is not None else block_size, T, K, rows.data_ptr(), rows.stride(0),
              _ptr(counts), _stream(topk_pos))
    return rows


# ---------------------------------------------------------------------------------------------- rows
def gather(src, rows, out, R=None, pcie=False):
    """out[i] = src[rows[i]] (zero row when rows[i] is outside [0, R)); src [R, row] uint8 (device or mapped host).
    pcie: src is pinned host memory; the copy then runs on a fixed 64-workgroup grid (spmla_gather_pcie)."""
    n = rows.shape[0]
    rowb = out.shape[-1]
    _need(rows.dtype == torch.int64 and rows.is_contiguous(), "rows int64 contiguous")
    _need(out.element_size() == 1 and out.dim() == 2 and out.stride(1) == 1 and out.shape[0] >= n,
          "out of bytes (uint8 / float8) [>= n, row] with contiguous rows")
    _lib.call("spmla_gather_pcie" if pcie else "spmla_gather", src.data_ptr() if torch.is_tensor(src) else int(src),
              int(R if R is not None else src.shape[0]), rowb, rows.data_ptr(), n, out.data_ptr(), out.stride(0),
              _stream(out))
    return out


def gather_tiers(src, rows, counts, out, R=None):
    """Host-tier staging: out[t * K + k] = src[rows[t, k]] for k < counts[t] (rows int32 [T, K], counts int32 [T]);
    other rows of out untouched (row 0 zeroed when counts[0] <= 0). src: pinned host memory (or HBM)."""
    T, K = rows.shape
    _need(rows.dtype == torch.int32 and rows.stride(1) == 1 and counts.dtype == torch.int32, "int32 rows / counts")
    _need(out.shape[0] >= T * K, "out holds T * K rows")
    _lib.call("spmla_gather_tiers", src.data_ptr() if torch.is_tensor(src) else int(src),
              int(R if R is not None else src.shape[0]), out.shape[-1], rows.data_ptr(), rows.stride(0),
              counts.data_ptr(), T, K, out.data_ptr(), out.stride(0), _stream(out))
    return out


def _dst_fmt(out):
    _need(out.dtype == torch.uint8 and out.shape[-1] in (ROW656, ROW576), "out rows: uint8 Row656 or Row576")
    return 0 if out.shape[-1] == ROW656 else 1


def row400_gather(src, rows, out, R=None, pcie=False):
    """out[i] = the GPU row (Row656 or Row576, by out's row width) of compact Row400 row src[rows[i]]; zero row when
    rows[i] is outside [0, R). src [R, 400] uint8 (pinned host memory with pcie=True, or HBM)."""
    n = rows.shape[0]
    _need(rows.dtype == torch.int64 and rows.is_contiguous(), "rows int64 contiguous")
    _need(out.element_size() == 1 and out.dim() == 2 and out.stride(1) == 1 and out.shape[0] >= n,
          "out of bytes (uint8 / float8) [>= n, row] with contiguous rows")
    _lib.call("spmla_row400_gather", src.data_ptr() if torch.is_tensor(src) else int(src),
              int(R if R is not None else src.shape[0]), rows.data_ptr(), n, out.data_ptr(), out.stride(0),
              _dst_fmt(out), int(bool(pcie)), _stream(out))
    return out


def row576_gather(src, rows, out, R=None):
    """out[i] = Row656 staging of Row576 row src[rows[i]] (codes as they are, scales 1.0, rope widened to bf16); zero
    row when rows[i] is outside [0, R). src [R, 576] uint8 (or a flat view of a paged cache), rows int64 [n]."""
    n = rows.numel()
    _need(rows.dtype == torch.int64 and rows.is_contiguous(), "rows int64 contiguous")
    _need(out.dtype == torch.uint8 and out.dim() == 2 and out.shape[1] == ROW656 and out.stride(1) == 1,
          "out [n, 656] uint8 rows")
    _need(out.shape[0] >= n, "out has fewer rows than rows")
    Rv = int(R if R is not None else src.shape[0])
    _lib.call("spmla_row576_gather", src.data_ptr(), Rv, rows.data_ptr(), n, out.data_ptr(), out.stride(0),
              _stream(out))
    return out


def row400_copy(src, src_rows, dst, dst_rows, R_src=None):
    """dst[dst_rows[i]] = the GPU row of Row400 row src[src_rows[i]] (pairs with an invalid side skipped)."""
    n = src_rows.shape[0]
    _need(src_rows.dtype == torch.int64 and dst_rows.dtype == torch.int64, "int64 rows")
    _lib.call("spmla_row400_copy", src.data_ptr() if torch.is_tensor(src) else int(src),
              int(R_src if R_src is not None else src.shape[0]), src_rows.data_ptr(), dst.data_ptr(), dst.shape[0],
              dst_rows.data_ptr(), n, _dst_fmt(dst), _stream(dst))


def row400_gather_tiers(src, rows, counts, out, R=None):
    """gather_tiers from compact Row400 host rows, decoded to out's row format (Row656 / Row576)."""
    T, K = rows.shape
    _need(rows.dtype == torch.int32 and rows.stride(1) == 1 and counts.dtype == torch.int32, "int32 rows / counts")
    _need(out.shape[0] >= T * K, "out holds T * K rows")
    _lib.call("spmla_row400_gather_tiers", src.data_ptr() if torch.is_tensor(src) else int(src),
              int(R if R is not None else src.shape[0]), rows.data_ptr(), rows.stride(0), counts.data_ptr(), T, K,
              out.data_ptr(), out.stride(0), _dst_fmt(out), _stream(out))
    return out


def row400_decode_tiers(src, rows, counts, out, R=None):
    """out row t * K + k = the GPU row (out's format: Row656 / Row576) of compact Row400 row src[rows[t, k]] in HBM
    for k < counts[t] (counts None: every k; zero row when outside [0, R)); other out rows untouched."""
    T, K = rows.shape
    _need(rows.dtype == torch.int32 and rows.stride(1) == 1, "int32 rows")
    _need(counts is None or counts.dtype == torch.int32, "int32 counts")
    _need(out.shape[0] >= T * K, "out holds T * K rows")
    _lib.call("spmla_row400_decode_tiers", src.data_ptr(), int(R if R is not None else src.shape[0]), rows.data_ptr(),
              rows.stride(0), _ptr(counts), T, K, out.data_ptr(), out.stride(0), _dst_fmt(out), _stream(out))
    return out


def copy_rows(src, src_rows, dst, dst_rows, R_src=None):
    n = src_rows.shape[0]
    _lib.call("spmla_copy_rows", src.data_ptr() if torch.is_tensor(src) else int(src),
              int(R_src if R_src is not None else src.shape[0]), src_rows.data_ptr(), dst.data_ptr(), dst.shape[0],
              dst_rows.data_ptr(), dst.shape[-1], n, _stream(dst))


class RowCache:
    """Device state of a dynamic W-way HBM row cache (spmla_wcache_*): C lines in S = C / W sets plus `cap` spill rows,
    both in one pool [C + cap, row_bytes] (Row656 lines that the attention reads, or compact Row400 lines that are
    decoded for it); tags, round-robin pointers, pins, and per host row the epoch of its last miss and that miss's
    pool row. Everything is zero-initialized once (tags -1); no buffer is cleared between steps. two=True: two-choice
    placement (a row may also live in a second, hashed set; every step and invalidation of this cache then uses
    both sets)."""

    def __init__(self, C, W, cap, device, two=False, row_bytes=ROW656):
        _need(C > 0 and W > 0 and C % W == 0 and cap >= 0, "RowCache: C a positive multiple of W, cap >= 0")
        _need(row_bytes in (ROW656, ROW400), "RowCache: Row656 or Row400 lines")
        self.C, self.W, self.S, self.cap = int(C), int(W), int(C) // int(W), int(cap)
        self.two = bool(two)
        self.device = torch.device(device)
        i32 = dict(dtype=torch.int32, device=self.device)
        self.tag = torch.full((self.C,), -1, **i32)
        self.rr = torch.zeros(self.S, **i32)
        self.cnt = torch.zeros(self.S, **i32)
        self.pin = torch.zeros(self.C, **i32)
        self.state = torch.zeros(4, **i32)              # epoch, misses, spill rows used, hits (of the last step)
        self.pool = torch.zeros((self.C + self.cap, int(row_bytes)), dtype=torch.uint8, device=self.device)
        self.n = 0
        self.R = 0

    def _tables(self, n, R):
        dev = self.device
        if R > self.R:
            self.claim = torch.zeros(R, dtype=torch.int32, device=dev)
            self.rdst = torch.zeros(R, dtype=torch.int32, device=dev)
            self.R = R
        if n > self.n:
            self.ml = torch.zeros(n, dtype=torch.int64, device=dev)
            self.mdst = torch.zeros(n, dtype=torch.int64, device=dev)
            self.n = n

    def set2(self, rows):
        """The second candidate set of each row (int64 tensor of rows >= 0) under two-choice placement."""
        return ((rows.long() * 2654435761) >> 12) % self.S

    def lookup(self, rows):
        """bool per row id (int64 tensor): currently in a cache line (diagnostics; no kernel of its own)."""
        tg = self.tag.view(self.S, self.W)
        r32 = rows[:, None].to(torch.int32)
        hit = (tg[(rows % self.S).long()] == r32).any(1)
        if self.two:
            hit |= (tg[self.set2(rows)] == r32).any(1)
        return hit & (rows >= 0)


def wcache_step(cache, idx, R, res=None):
    """One decode step of the row cache for idx [T, K] int32 host rows -> res [T, K] int32: the pool row of each
    entry (line or C + spill row), -2 for a row left on the host (spill area full), -1 invalid."""
    T, K = idx.shape
    _need(idx.dtype == torch.int32 and idx.stride(1) == 1, "idx int32 [T, K]")
    cache._tables(T * K, int(R))
    if res is None:
        res = torch.empty(T, K, dtype=torch.int32, device=idx.device)
    _lib.call("spmla_wcache_step", *_wc_args(cache, idx, R), res.data_ptr(), res.stride(0), _stream(idx))
    return res


def _wc_args(cache, idx, R):
    T, K = idx.shape
    return (idx.data_ptr(), idx.stride(0), T, K, int(R), cache.tag.data_ptr(), cache.C, cache.W, cache.rr.data_ptr(),
            cache.cnt.data_ptr(), cache.pin.data_ptr(), cache.claim.data_ptr(), cache.rdst.data_ptr(),
            cache.ml.data_ptr(), cache.mdst.data_ptr(), cache.state.data_ptr(), cache.cap, int(cache.two))


def wcache_place(cache, idx, R):
    """First half of wcache_step: lookup and placement (the miss list and tags are final; wcache_fill may follow)."""
    T, K = idx.shape
    _need(idx.dtype == torch.int32 and idx.stride(1) == 1, "idx int32 [T, K]")
    cache._tables(T * K, int(R))
    _lib.call("spmla_wcache_place", *_wc_args(cache, idx, R), _stream(idx))


def wcache_resolve(cache, idx, R, res=None):
    """Second half of wcache_step: res [T, K] and the round-robin advance."""
    T, K = idx.shape
    if res is None:
        res = torch.empty(T, K, dtype=torch.int32, device=idx.device)
    _lib.call("spmla_wcache_resolve", *_wc_args(cache, idx, R), res.data_ptr(), res.stride(0), _stream(idx))
    return res


def wcache_fill(cache, host, R, host_fmt, n):
    """The step's row copies from the host pool (Row656 = host_fmt 0, compact Row400 = 2) into cache.pool (Row656
    lines, or compact Row400 lines that take Row400 rows as they are); n = the step's entry count (bounds the miss
    list)."""
    pool_fmt = 2 if cache.pool.shape[1] == ROW400 else 0
    _lib.call("spmla_wcache_fill", host.data_ptr() if torch.is_tensor(host) else int(host), int(R), int(host_fmt),
              pool_fmt, cache.ml.data_ptr(), cache.mdst.data_ptr(), cache.state.data_ptr(), int(n),
              cache.pool.data_ptr(), cache.pool.shape[0], _stream(cache.pool))


def wcache_invalidate(cache, slots, R):
    _need(slots.dtype == torch.int64, "slots int64")
    _lib.call("spmla_wcache_invalidate", slots.data_ptr(), slots.shape[0], int(R), cache.tag.data_ptr(), cache.C,
              cache.W, int(cache.two), _stream(slots))


def split_res(idx, res, hbm=None, hbm_cnt=None, host=None, host_cnt=None):
    T, K = idx.shape
    dev = idx.device
    hbm = torch.empty(T, K, dtype=torch.int32, device=dev) if hbm is None else hbm
    host = torch.empty(T, K, dtype=torch.int32, device=dev) if host is None else host
    hbm_cnt = torch.empty(T, dtype=torch.int32, device=dev) if hbm_cnt is None else hbm_cnt
    host_cnt = torch.empty(T, dtype=torch.int32, device=dev) if host_cnt is None else host_cnt
    _lib.call("spmla_split_res", idx.data_ptr(), idx.stride(0), res.data_ptr(), res.stride(0), T, K, hbm.data_ptr(),
              hbm.stride(0), hbm_cnt.data_ptr(), host.data_ptr(), host.stride(0), host_cnt.data_ptr(), _stream(idx))
    return hbm, hbm_cnt, host, host_cnt


def wcache_split(cache, res, hit=None, hit_cnt=None, fresh=None, fresh_cnt=None):
    """Entries of a cache step's res [T, K] split into this step's hits and the rows its fill brings in (pool rows,
    compacted per token, -1 padded, counts per token)."""
    T, K = res.shape
    dev = res.device
    hit = torch.empty(T, K, dtype=torch.int32, device=dev) if hit is None else hit
    fresh = torch.empty(T, K, dtype=torch.int32, device=dev) if fresh is None else fresh
    hit_cnt = torch.empty(T, dtype=torch.int32, device=dev) if hit_cnt is None else hit_cnt
    fresh_cnt = torch.empty(T, dtype=torch.int32, device=dev) if fresh_cnt is None else fresh_cnt
    _lib.call("spmla_wcache_split", res.data_ptr(), res.stride(0), T, K, cache.pin.data_ptr(), cache.C,
              cache.state.data_ptr(), hit.data_ptr(), hit.stride(0), hit_cnt.data_ptr(), fresh.data_ptr(),
              fresh.stride(0), fresh_cnt.data_ptr(), _stream(res))
    return hit, hit_cnt, fresh, fresh_cnt


def tier_split(idx, rowmap, R, hbm=None, hbm_cnt=None, host=None, host_cnt=None):
    T, K = idx.shape
    dev = idx.device
    hbm = torch.empty(T, K, dtype=torch.int32, device=dev) if hbm is None else hbm
    host = torch.empty(T, K, dtype=torch.int32, device=dev) if host is None else host
    hbm_cnt = torch.empty(T, dtype=torch.int32, device=dev) if hbm_cnt is None else hbm_cnt
    host_cnt = torch.empty(T, dtype=torch.int32, device=dev) if host_cnt is None else host_cnt
    _lib.call("spmla_tier_split", idx.data_ptr(), idx.stride(0), T, K, rowmap.data_ptr(), int(R), hbm.data_ptr(),
              hbm.stride(0), hbm_cnt.data_ptr(), host.data_ptr(), host.stride(0), host_cnt.data_ptr(), _stream(idx))
    return hbm, hbm_cnt, host, host_cnt


def compact_stage(rows, sidx, workspace=None):
    """rows [tot] int64, sidx [M, K] int32 -> (sel [tot] int64 (first U valid), U [1] int32 on device, sidx2)."""
    tot = rows.shape[0]
    M, K = sidx.shape
    W = (tot + 31) // 32
    if workspace is None:
        workspace = torch.empty(max(1, 2 * W), dtype=torch.int32, device=rows.device)
    sel = torch.empty(max(1, tot), dtype=torch.int64, device=rows.device)
    U = torch.empty(1, dtype=torch.int32, device=rows.device)
    sidx2 = torch.empty_like(sidx)
    _lib.call("spmla_compact_stage", rows.data_ptr(), tot, sidx.data_ptr(), sidx.stride(0), M, K,
              workspace.data_ptr(), sel.data_ptr(), U.data_ptr(), sidx2.data_ptr(), sidx2.stride(0), _stream(rows))
    return sel, U, sidx2


# ---------------------------------------------------------------------------------------------- attention
def attention_ok(q, idx):
    """Preconditions of spmla_attn_splitk (the reference's offload_cuda2.ok analogue)."""
    return (q.dtype == torch.bfloat16 and q.dim() == 3 and q.shape[2] == D_QK and q.stride(2) == 1
            and q.data_ptr() % 16 == 0 and q.stride(0) % 8 == 0 and q.stride(1) % 8 == 0
            and idx.dtype == torch.int32 and idx.stride(1) == 1)


ATTN_SPLIT_ROWS = 2048      # rows of one (token, split) in spmla_attn's split merge, rounded up to 32-row tiles


def auto_split(T, H, K, cus=256):
    """Row splits per token. 1 when the unsplit launch has at least cus * 3 / 8 workgroups of 32 heads (the
    head-group kernel: a workgroup of 32 heads over all K rows takes as long as one of 128 heads over K / 4 rows, so
    a partly filled unsplit launch still beats a split one with its merge); else the in-kernel split merge over
    128-head workgroups, doubled while that launch has fewer workgroups than compute units and every split keeps
    at least 8 tiles of 32 rows (at most 8 splits). 1 as well when a split would hold more than ATTN_SPLIT_ROWS
    rows (the split kernel's limit; the head-group kernel takes any K)."""
    if T * ((H + 31) // 32) * 8 >= cus * 3:
        return 1
    n = T * ((H + 127) // 128)
    s = 1
    while s < 8 and n * s < cus and K >= 2 * s * 256:
        s *= 2
    if -(-(-(-K // s)) // 32) * 32 > ATTN_SPLIT_ROWS:
        return 1
    return s


def auto_split576(T, H, K, cus=256):
    """Row splits per token of a Row576 launch (one kernel, 32 heads per workgroup; split partials in fp32, merged by
    spmla_lse_merge): doubled while the launch has fewer than cus * 3 / 8 workgroups and every split keeps at least
    8 tiles of 32 rows (at most 8 splits)."""
    n = T * ((H + 31) // 32)
    s = 1
    while s < 8 and n * s * 8 < cus * 3 and K >= 2 * s * 256:
        s *= 2
    return s


def attn_ws_bytes(T, H, split):
    """Bytes of the workspace attend needs for T tokens, H heads and `split` splits (0 for split 1)."""
    return int(_lib.lib().spmla_attn_ws_bytes(T, H, split))


def attend(q, pool, idx, sm_scale, kv_scale=1.0, out=None, lse=None, split=None, kcount=None, ws=None, R=None,
           row_bytes=None):
    """q [T, H, 576] bf16, pool [R, 656] uint8 Row656 rows (or a mapped host address with R given), idx [T, K]
    int32 rows -> (out [T, H, 512] bf16, lse [T, H] fp32). Row576 rows (pool [..., 576], or row_bytes=576: the
    per-tensor fp8 cache, every code times kv_scale) go to spmla_attn576, whose splits merge through fp32 partials
    (split None: auto_split576). For Row656, split > 1 (at most 8) cuts K into partials that the
    kernel merges (spmla_attn; ws: a uint8 workspace of attn_ws_bytes whose leading counter bytes are zero -- the
    kernel leaves them so --, else a cached one per stream; under HIP graph capture either ws or a workspace reserved
    by an earlier eager call, see reserve_workspace); None: auto_split."""
    T, H, _ = q.shape
    K = idx.shape[1]
    rb = int(row_bytes) if row_bytes is not None else (int(pool.shape[-1]) if torch.is_tensor(pool) else ROW656)
    _need(rb in (ROW656, ROW576), "attend: Row656 or Row576 rows")
    if split is None:
        split = auto_split576(T, H, K) if rb == ROW576 else auto_split(T, H, K)
    _need(attention_ok(q, idx), "attend: q must be bf16 [T, H, 576] with 16-byte aligned rows, idx int32")
    if out is None:
        out = torch.empty(T, H, D_LAT, dtype=torch.bfloat16, device=q.device)
    if lse is None:
        lse = torch.empty(T, H, dtype=torch.float32, device=q.device)
    Rv = int(R if R is not None else pool.shape[0])
    pptr = pool.data_ptr() if torch.is_tensor(pool) else int(pool)
    st = _stream(q)
    if rb == ROW576:
        _need(1 <= split <= 8, "attend: split must be 1 .. 8")
        if split == 1:
            _lib.call("spmla_attn576", q.data_ptr(), q.stride(0), q.stride(1), pptr, Rv, idx.data_ptr(),
                      idx.stride(0), K, _ptr(kcount), T, H, float(sm_scale), float(kv_scale), 1, out.data_ptr(),
                      out.stride(0), out.stride(1), lse.data_ptr(), lse.stride(0), None, None, st)
            return out, lse
        opart = torch.empty(split, T, H, D_LAT, dtype=torch.float32, device=q.device)
        lpart = torch.empty(split, T, H, dtype=torch.float32, device=q.device)
        _lib.call("spmla_attn576", q.data_ptr(), q.stride(0), q.stride(1), pptr, Rv, idx.data_ptr(), idx.stride(0),
                  K, _ptr(kcount), T, H, float(sm_scale), float(kv_scale), split, None, 0, 0, None, 0,
                  opart.data_ptr(), lpart.data_ptr(), st)
        return lse_merge(opart, lpart, out=out, lse=lse)
    if split == 1:
        _lib.call("spmla_attn_splitk", q.data_ptr(), q.stride(0), q.stride(1), pptr, Rv, idx.data_ptr(),
                  idx.stride(0), K, _ptr(kcount), T, H, float(sm_scale), float(kv_scale), 1, out.data_ptr(),
                  out.stride(0), out.stride(1), lse.data_ptr(), lse.stride(0), None, None, st)
        return out, lse
    _need(1 <= split <= 8, "attend: split must be 1 .. 8")
    nb = int(_lib.lib().spmla_attn_ws_bytes(T, H, split))
    if ws is None:
        ws, key = _workspace("attn", q.device, nb, zero=True)
        cnt = _attn_counter_bytes(T, H)
        if key is None:                   # captured: replays come in any order, so every replay clears its counters
            ws[:cnt].zero_()
        else:
            if cnt > _WS_CNT[key]:        # counter bytes the previous launch used as scratch: cleared by a fill kernel
                ws[_WS_CNT[key]:cnt].zero_()
            _WS_CNT[key] = cnt
    _need(ws.dtype == torch.uint8 and ws.numel() >= nb, "attend: workspace too small")
    _lib.call("spmla_attn", q.data_ptr(), q.stride(0), q.stride(1), pptr, Rv, idx.data_ptr(), idx.stride(0), K,
              _ptr(kcount), T, H, float(sm_scale), float(kv_scale), split, out.data_ptr(), out.stride(0),
              out.stride(1), lse.data_ptr(), lse.stride(0), ws.data_ptr(), ws.numel(), st)
    return out, lse


def attend_partial(q, pool, idx, sm_scale, kv_scale=1.0, opart=None, lpart=None, split=1, kcount=None, R=None,
                   row_bytes=None):
    """Like attend, but the result stays as `split` normalized fp32 partials (opart [split, T, H, 512], lpart
    [split, T, H]) for a later lse_merge (tier partials use split = 1). Row576 pools (pool [..., 576] or
    row_bytes=576) go to spmla_attn576."""
    T, H, _ = q.shape
    K = idx.shape[1]
    _need(attention_ok(q, idx), "attend_partial: q must be bf16 [T, H, 576] with 16-byte aligned rows, idx int32")
    if opart is None:
        opart = torch.empty(split, T, H, D_LAT, dtype=torch.float32, device=q.device)
    if lpart is None:
        lpart = torch.empty(split, T, H, dtype=torch.float32, device=q.device)
    _need(opart.is_contiguous() and lpart.is_contiguous() and opart.shape[:3] == (split, T, H), "partials layout")
    Rv = int(R if R is not None else pool.shape[0])
    pptr = pool.data_ptr() if torch.is_tensor(pool) else int(pool)
    rb = int(row_bytes) if row_bytes is not None else (int(pool.shape[-1]) if torch.is_tensor(pool) else ROW656)
    _need(rb in (ROW656, ROW576), "attend_partial: Row656 or Row576 rows")
    _lib.call("spmla_attn576" if rb == ROW576 else "spmla_attn_splitk", q.data_ptr(), q.stride(0), q.stride(1), pptr,
              Rv, idx.data_ptr(), idx.stride(0), K, _ptr(kcount), T, H, float(sm_scale), float(kv_scale), split, None,
              0, 0, None, 0, opart.data_ptr(), lpart.data_ptr(), _stream(q))
    return opart, lpart


def attend_merge(q, pool, idx, sm_scale, kv_scale, prior_o, prior_lse, out=None, lse=None, kcount=None, R=None):
    """attend, merged with a prior normalized partial (prior_o [T, H, 512] fp32, prior_lse [T, H]) of the same tokens
    and heads in the kernel's epilogue: the two-tier decode step's second tier without a separate lse_merge."""
    T, H, _ = q.shape
    K = idx.shape[1]
    _need(attention_ok(q, idx), "attend_merge: q must be bf16 [T, H, 576] with 16-byte aligned rows, idx int32")
    _need(prior_o.dtype == torch.float32 and prior_o.shape == (T, H, D_LAT) and prior_o.stride(2) == 1,
          "prior_o fp32 [T, H, 512]")
    _need(prior_lse.dtype == torch.float32 and prior_lse.shape == (T, H) and prior_lse.stride(1) == 1, "prior_lse")
    if out is None:
        out = torch.empty(T, H, D_LAT, dtype=torch.bfloat16, device=q.device)
    if lse is None:
        lse = torch.empty(T, H, dtype=torch.float32, device=q.device)
    Rv = int(R if R is not None else pool.shape[0])
    pptr = pool.data_ptr() if torch.is_tensor(pool) else int(pool)
    _lib.call("spmla_attn_merge", q.data_ptr(), q.stride(0), q.stride(1), pptr, Rv, idx.data_ptr(), idx.stride(0), K,
              _ptr(kcount), T, H, float(sm_scale), float(kv_scale), prior_o.data_ptr(), prior_o.stride(0),
              prior_o.stride(1), prior_lse.data_ptr(), prior_lse.stride(0), out.data_ptr(), out.stride(0),
              out.stride(1), lse.data_ptr(), lse.stride(0), _stream(q))
    return out, lse


def lse_merge(parts, lses, out=None, out_f32=None, lse=None):
    """parts [n, T, H, 512] fp32 or bf16 (any strides with contiguous rows), lses [n, T, H] -> merged (out, lse)."""
    n, T, H, _ = parts.shape
    if out is None and out_f32 is None:
        out = torch.empty(T, H, D_LAT, dtype=torch.bfloat16, device=parts.device)
    if lse is None:
        lse = torch.empty(T, H, dtype=torch.float32, device=parts.device)
    ref = out if out is not None else out_f32
    if out is not None and out_f32 is not None:
        _need(out.stride() == out_f32.stride(), "out and out_f32 need the same strides")
    _lib.call("spmla_lse_merge", parts.data_ptr(), int(parts.dtype == torch.bfloat16), parts.stride(0),
              parts.stride(1), parts.stride(2), lses.data_ptr(), lses.stride(0), lses.stride(1), n, T, H,
              _ptr(out), ref.stride(0), ref.stride(1), _ptr(out_f32), lse.data_ptr(), lse.stride(0),
              _stream(parts))
    return (out if out is not None else out_f32), lse


# ---------------------------------------------------------------------------------------------- MLA absorbed matmuls
def bmm_fp8(a, codes, scales, scale_k, out):
    """out[n, b, j] = sum_k a[n, b, k] * bf16(codes[n, j, k] (e4m3) * S), S = scales[n, j, k // 128] (scale_k) else
    scales[n, k, j // 128]; a bf16 [N, B, K] (any strides), out bf16 or fp32 [N, B, J] (any strides)."""
    N, B, K = a.shape
    J = codes.shape[1]
    _need(a.dtype == torch.bfloat16, "a must be bf16")
    _need(codes.dtype in (torch.uint8, torch.float8_e4m3fn) and codes.shape[0] == N and codes.shape[2] == K,
          "codes [N, J, K] e4m3")
    _need(scales.dtype == torch.float32, "scales fp32")
    _need(out.dtype in (torch.bfloat16, torch.float32) and tuple(out.shape) == (N, B, J), "out [N, B, J]")
    _lib.call("spmla_bmm_fp8", a.data_ptr(), a.stride(0), a.stride(1), a.stride(2), codes.data_ptr(), codes.stride(0),
              codes.stride(1), codes.stride(2), scales.data_ptr(), scales.stride(0), scales.stride(1),
              scales.stride(2), int(bool(scale_k)), out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
              int(out.dtype == torch.float32), N, B, J, K, _stream(a))
    return out


def mla_query(q_nope, q_pe, codes_uk, scales_uk, out=None):
    """The decode query of the sparse attention in one launch: out[t, h, :512] = q_nope[t, h] @ W_UK_T[h] (FP8
    weights, codes [H, 512, 128], scales [H, 128, 4]), out[t, h, 512:] = q_pe[t, h]."""
    T, H, _ = q_nope.shape
    _need(q_nope.dtype == torch.bfloat16 and q_nope.shape[2] == 128 and q_nope.stride(2) == 1, "q_nope [T, H, 128]")
    _need(q_pe.dtype == torch.bfloat16 and tuple(q_pe.shape) == (T, H, 64) and q_pe.stride(2) == 1, "q_pe [T, H, 64]")
    _need(tuple(codes_uk.shape) == (H, 512, 128) and codes_uk.is_contiguous(), "codes_uk [H, 512, 128]")
    _need(tuple(scales_uk.shape) == (H, 128, 4) and scales_uk.is_contiguous() and scales_uk.dtype == torch.float32,
          "scales_uk [H, 128, 4] fp32")
    if out is None:
        out = torch.empty(T, H, D_QK, dtype=torch.bfloat16, device=q_nope.device)
    _need(out.dtype == torch.bfloat16 and tuple(out.shape) == (T, H, D_QK) and out.stride(2) == 1, "out [T, H, 576]")
    _lib.call("spmla_mla_query", q_nope.data_ptr(), q_nope.stride(0), q_nope.stride(1), q_pe.data_ptr(),
              q_pe.stride(0), q_pe.stride(1), codes_uk.data_ptr(), scales_uk.data_ptr(), T, H, out.data_ptr(),
              out.stride(0), out.stride(1), _stream(q_nope))
    return out


def topk_overlap(sets):
    """sets: int32 [L, n, K] top-k rows of L layers (-1 = none) -> (hits [L, L, n] int32: valid entries of layer b
    also in layer a, diagonal 0; nvalid [L, n] int32)."""
    _need(sets.dtype == torch.int32 and sets.dim() == 3 and sets.stride(2) == 1, "topk_overlap: int32 [L, n, K]")
    L, n, K = sets.shape
    hits = torch.zeros(L, L, n, dtype=torch.int32, device=sets.device)
    nvalid = torch.empty(L, n, dtype=torch.int32, device=sets.device)
    _lib.call("spmla_topk_overlap", sets.data_ptr(), sets.stride(0), sets.stride(1), L, n, K, hits.data_ptr(),
              nvalid.data_ptr(), _stream(sets))
    return hits, nvalid


def mtp_union(idx, ql=None, cu=None, R=None, nmax=None, max_query_len=None):
    """The union of each request's MTP top-k rows with token masks: idx [T, topk] int32 rows, requests of ql tokens
    (or boundaries cu [nreq + 1] on the device, with max_query_len, the host-known largest request, at most 6: the
    boundaries themselves are not read back) -> (u [nreq, nmax] int32 (-1 padded), mk [nreq, nmax] uint8, cnt [nreq]
    int32), rows ordered by mask descending then first occurrence (the request-packed decode's row list). A request
    longer than 6 tokens is a caller error the kernel does not see: it uses the first 6."""
    T, topk = idx.shape
    _need(idx.dtype == torch.int32 and idx.stride(1) == 1, "idx int32 [T, topk]")
    _need(R is not None, "mtp_union: R (rows of the pool) is required")
    if cu is not None:
        _need(max_query_len is not None, "mtp_union: cu needs max_query_len (the largest request, host-known)")
        _need(0 <= int(max_query_len) <= 6, "mtp_union: at most 6 tokens per request")
        cu = cu.to(torch.int32).contiguous()
        nreq, ql_ = cu.shape[0] - 1, 0
        gmax = 6
    else:
        _need(ql is not None and 0 < ql <= 6, "mtp_union: ql (1 .. 6) or cu")
        nreq, ql_ = (T + ql - 1) // ql, int(ql)
        gmax = min(ql, 6)
    if nmax is None:
        nmax = max(1, gmax * topk)
    u = torch.empty(nreq, nmax, dtype=torch.int32, device=idx.device)
    mk = torch.zeros(nreq, nmax, dtype=torch.uint8, device=idx.device)
    cnt = torch.empty(nreq, dtype=torch.int32, device=idx.device)
    _lib.call("spmla_mtp_union", idx.data_ptr(), idx.stride(0), T, ql_, _ptr(cu), nreq, int(R), topk, nmax,
              u.data_ptr(), mk.data_ptr(), cnt.data_ptr(), _stream(idx))
    return u, mk, cnt


def attend_packed(q, pool, idx, sm_scale, kv_scale=1.0, ql=None, cu=None, out=None, lse=None, split=1, tpg=None,
                  union=None, max_query_len=None):
    """Request-packed MTP decode (the reference's ARC_OFFLOAD_CUDA_PK path): the tokens of a request (ql tokens each,
    or boundaries cu) attend over the union of their top-k rows (mtp_union), each union row loaded and converted once
    per request and head group, each token's softmax kept to its own rows. Same result as attend per token up to the
    fp32 summation order. q [T, H, 576] bf16, pool Row656 rows, idx [T, K] int32 -> (out [T, H, 512] bf16, lse).
    With cu, max_query_len is the host-known largest request (at most 6)."""
    T, H, _ = q.shape
    _need(attention_ok(q, idx), "attend_packed: q must be bf16 [T, H, 576] with 16-byte aligned rows, idx int32")
    R = int(pool.shape[0])
    _need(cu is not None or (ql is not None and 0 < ql <= 6), "attend_packed: ql (1 .. 6) or cu")
    u, mk, cnt = union if union is not None else mtp_union(idx, ql=ql, cu=cu, R=R, max_query_len=max_query_len)
    nreq, nmax = u.shape
    if tpg is None:
        g = min(int(ql), 6) if cu is None else min(int(max_query_len or 6), 6)
        tpg = 1 if g <= 1 else (2 if g <= 2 else (4 if g <= 4 else 8))
    if out is None:
        out = torch.empty(T, H, D_LAT, dtype=torch.bfloat16, device=q.device)
    if lse is None:
        lse = torch.empty(T, H, dtype=torch.float32, device=q.device)
    cu_t = cu.to(torch.int32).contiguous() if cu is not None else None
    st = _stream(q)
    if split == 1:
        _lib.call("spmla_attn_packed", q.data_ptr(), q.stride(0), q.stride(1), pool.data_ptr(), R, u.data_ptr(),
                  mk.data_ptr(), cnt.data_ptr(), nmax, _ptr(cu_t), int(ql or 0), nreq, T, H, tpg, float(sm_scale),
                  float(kv_scale), 1, out.data_ptr(), out.stride(0), out.stride(1), lse.data_ptr(), lse.stride(0),
                  None, None, st)
        return out, lse
    opart = torch.empty(split, T, H, D_LAT, dtype=torch.float32, device=q.device)
    lpart = torch.empty(split, T, H, dtype=torch.float32, device=q.device)
    _lib.call("spmla_attn_packed", q.data_ptr(), q.stride(0), q.stride(1), pool.data_ptr(), R, u.data_ptr(),
              mk.data_ptr(), cnt.data_ptr(), nmax, _ptr(cu_t), int(ql or 0), nreq, T, H, tpg, float(sm_scale),
              float(kv_scale), split, None, 0, 0, None, 0, opart.data_ptr(), lpart.data_ptr(), st)
    lse_merge(opart, lpart, out=out, lse=lse)
    return out, lse
