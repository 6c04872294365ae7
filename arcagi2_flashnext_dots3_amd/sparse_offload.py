"""Host-offloaded sparse-MLA KV rows for one DSA layer: the LayerOffload interface of the reference
(dotsnote/engine/arcstats_pkg/arcstats/sparse_offload.py:1051-1648) on libspmla_gfx950.so.

Tiers
  host pool   [R, 656] uint8 Row656 rows in pinned host memory (torch's pinned allocator = hipHostMalloc; the kernels
              read and write it through its device-visible address, 16-byte accesses over PCIe). This replaces the
              reference's cudaHostRegister'ed buffer (_HostReg, sparse_offload.py:917-980). With row_fmt="e2m2" the
              pool holds the reference's compact Row400 rows instead (offload_rowfmt.py, ARC_OFFLOAD_ROW_FMT=e2m2):
              every host read decodes them into Row656 on the way, so 39% fewer bytes cross PCIe per row.
  HBM cache   [C, 656] uint8 hot rows with tag[line] = host row and rowmap[row] = line (-1 = host only). Two modes:
              cache_mode="static": the hot set is chosen by the caller (set_hot_rows, e.g. hot_rows_by_frequency over
              recent selections); cache_mode="ways": the reference's dynamic W-way set-associative cache
              (sparse_offload.py:677-789, :1595-1622): every attend() looks its rows up, gives the distinct misses
              lines (round-robin over the unpinned ways of the row's set) or spill rows, copies them in over PCIe
              and attends the whole step from HBM.

Decode (attend): the selected host rows of each token are split by tier (spmla_tier_split: cache hits -> lines,
misses -> host rows, both compacted in order); the HBM tier is attended in place into an fp32 partial (o, lse); the
host tier's rows are first copied over PCIe into an HBM staging area (spmla_gather_tiers, the reference's miss fill)
and attended there by spmla_attn_merge, which merges the HBM tier's partial exactly in its epilogue (the
reference's tier combine). Without a cache (C = 0) every row takes the host tier.
"""
import os
import re

import torch

from . import kernels
from .diagnostics import AccessTrace, AttnTimer

ROW = kernels.ROW656
HOST_ROW = {"row656": kernels.ROW656, "e2m2": kernels.ROW400}


def host_memory_available():
    """Bytes of host memory the kernel reports available (MemAvailable of /proc/meminfo), None when unknown."""
    try:
        with open("/proc/meminfo") as fh:
            for line in fh:
                if line.startswith("MemAvailable:"):
                    return int(line.split()[1]) * 1024
    except OSError:
        pass
    return None


def check_host_budget(nbytes, available=None):
    """Refuse a pinned host pool larger than a fraction of the available host memory (ARC_OFFLOAD_HOST_FRAC, default
    0.5): pinned pages stay resident, so an oversized pool would exhaust the host instead of failing here (the
    reference's guard, sparse_offload.py:925-932)."""
    frac = float(os.environ.get("ARC_OFFLOAD_HOST_FRAC", "0.5"))
    avail = host_memory_available() if available is None else available
    if avail and nbytes > frac * avail:
        raise RuntimeError(f"offload host pool of {nbytes / 2**30:.1f} GiB exceeds {frac:.0%} of the "
                           f"{avail / 2**30:.1f} GiB of available host memory: give the layer fewer host rows "
                           f"(or raise ARC_OFFLOAD_HOST_FRAC)")


def hot_rows_by_frequency(counts, C):
    """Rows to keep in an HBM cache of C lines: the C most frequently selected rows (counts [R] int64 selection
    counts), equal counts -> lower row id first; rows never selected are not taken."""
    C = min(int(C), counts.shape[0])
    order = torch.sort(-counts.to(torch.int64), stable=True).indices[:C]
    return order[counts[order] > 0]


class LayerOffload:
    """One DSA layer's offloaded KV rows (reference LayerOffload, sparse_offload.py:1051).

    num_host_rows: R, the number of cache slots (every slot id written by store() is a host row id);
    device: the GPU; key: the layer's cache prefix (identification only); cache_rows: C lines of HBM hot-row cache;
    row_fmt: "row656" (host rows as the GPU reads them) or "e2m2" (the reference's compact Row400 host rows,
    offload_rowfmt.py:1-22; values = code * kv_scale, so store and attend take the same kv_scale);
    cache_mode: "static" (set_hot_rows) or "ways" (dynamic W-way cache with `ways` lines per set, C % ways == 0, and
    `spill_rows` HBM rows for misses that find no free way; a step with more entries than spill rows can leave rows on
    the host, which then take the host tier). overlap_fill (ways): attend over the step's hits on a second stream while
    the misses are copied in, then over the fresh rows with the hits' partial merged in the epilogue; False: one
    attention over the whole step after the copy (bit-identical to attending the gathered rows). cache_fmt (static,
    row_fmt="e2m2"): "row656" lines decoded once when filled, or "e2m2": the reference's compact GPU row cache
    (offload_rowfmt.py:1-22 with its compact cache lines, csrc/offload_attn2.cu:210-256), Row400 lines in HBM (39%
    fewer bytes per line) whose selected lines are decoded into Row656 staging each step before the HBM-tier
    attention (same values, bit-identical results); with cache_mode="ways" the W-way pool holds Row400 lines the same
    way (misses copied in as they are, the step's pool rows decoded into staging for the attention). two_choice (ways):
    the reference's two-choice set placement (ARC_OFFLOAD_TWO_CHOICE, offload_fill.py:16-23): a missing row whose set
    has no free way takes one in a second, hashed set before it spills; lookups and invalidations cover both sets.
    trace: a diagnostics.AccessTrace that records the stored slots and the decode rows of a window of calls.
    stats_every=N: every N attend calls, `log` gets the cache's hit rate over that call's rows. lstats_every=N (W-way
    cache): every N calls, that call's hits, distinct misses and spill rows.
    """

    _count = 0           # layers built in this process (the first one takes the default access trace)

    def __init__(self, num_host_rows, device, key=None, cache_rows=0, row_fmt="row656", cache_mode="static", ways=16,
                 spill_rows=131072, overlap_fill=True, two_choice=False, cache_fmt="row656", packed=False,
                 time_every=None, host_direct=False, trace=None, stats_every=None, log=print, lstats_every=None):
        if row_fmt not in HOST_ROW:
            raise ValueError(f"row_fmt must be one of {sorted(HOST_ROW)}")
        if cache_mode not in ("static", "ways"):
            raise ValueError("cache_mode must be 'static' or 'ways'")
        if packed and (cache_mode != "static" or cache_fmt != "row656"):
            raise ValueError("packed=True takes the static hot set with Row656 lines (or no cache)")
        if host_direct and (cache_mode != "static" or row_fmt != "row656" or cache_fmt != "row656"):
            raise ValueError("host_direct=True takes Row656 host rows and the static hot set")
        self.R = int(num_host_rows)
        self.device = torch.device(device)
        self.key = key
        self.row_fmt = row_fmt
        check_host_budget(self.R * HOST_ROW[row_fmt])
        self.host = torch.zeros((self.R, HOST_ROW[row_fmt]), dtype=torch.uint8, pin_memory=True)
        self.C = min(int(cache_rows), self.R)
        if cache_fmt not in HOST_ROW or (cache_fmt == "e2m2" and row_fmt != "e2m2"):
            raise ValueError("cache_fmt 'e2m2' needs row_fmt='e2m2'")
        self.cache_fmt = cache_fmt
        self.cache = torch.zeros((max(self.C, 1) if cache_mode == "static" else 1, HOST_ROW[cache_fmt]),
                                 dtype=torch.uint8, device=self.device)
        self.tag = torch.full((max(self.C, 1),), -1, dtype=torch.int64, device=self.device)
        self.rowmap = torch.full((max(self.R, 1),), -1, dtype=torch.int32, device=self.device)
        self._ws = {}
        self.mode = cache_mode
        self.overlap_fill = bool(overlap_fill)
        # request-packed MTP decode for ql > 1 (the reference's ARC_OFFLOAD_CUDA_PK, sparse_offload.py:1456-1515)
        self.packed = bool(packed)
        # host-tier rows read by the attention in place over PCIe (the reference's loaders fetch misses inside the
        # attention, csrc/offload_attn2.cu:177-208), instead of a staging copy into HBM first
        self.host_direct = bool(host_direct)
        # GPU-event timing of every attend call, printed every N calls (ARC_OFFLOAD_ATTN2_TIME=N; 0: off)
        if time_every is None:
            time_every = int(os.environ.get("ARC_OFFLOAD_ATTN2_TIME", "0") or 0)
        self.timer = AttnTimer(time_every)
        # stored slots and decode rows over a window of calls to an .npz (diagnostics.AccessTrace; None: taken from
        # ARC_OFFLOAD_DUMP / ARC_OFFLOAD_DUMP_LAYERS, where the first layer built in the process is the default one)
        self.trace = trace if trace is not None else AccessTrace.from_env(key, self.device,
                                                                         first=LayerOffload._count == 0)
        LayerOffload._count += 1
        # the cache's hit rate over the step's rows as attend finds it, logged every N calls (ARC_OFFLOAD_STATS=N,
        # sparse_offload.py:1540-1550; a host synchronization per logged call)
        if stats_every is None:
            stats_every = int(os.environ.get("ARC_OFFLOAD_STATS", "0") or 0)
        self.stats_every = int(stats_every)
        self.log = log
        self._ncall = 0
        # the W-way cache's counts of each call (hits, distinct misses, spill rows), logged every N calls
        # (ARC_OFFLOAD_LSTATS=N, sparse_offload.py:210-211, :1302-1309; reads them back: a host synchronization)
        if lstats_every is None:
            lstats_every = int(os.environ.get("ARC_OFFLOAD_LSTATS", "0") or 0)
        self.lstats_every = int(lstats_every)
        self._lcall = 0
        m = re.search(r"layers\.(\d+)\.", key or "")
        self.layer = int(m.group(1)) if m else -1         # backbone layer id from the cache key, as the reference
        self.wc = None
        self.W = int(ways) if cache_mode == "ways" else 1
        if cache_mode == "ways":
            if self.C <= 0 or self.C % int(ways):
                raise ValueError("cache_mode='ways' needs cache_rows a positive multiple of ways")
            self.wc = kernels.RowCache(self.C, int(ways), int(spill_rows), self.device, two=two_choice,
                                       row_bytes=HOST_ROW[cache_fmt])

    # ------------------------------------------------------------------------------------------------ rows in
    def store(self, kv_c_normed, k_pe, slots, kv_scale=1.0):
        """Quantize-and-pack n tokens (kv_c_normed [n, 512] bf16, k_pe [n, 64] / [n, 1, 64] bf16) into host rows
        `slots` [n] int64 (reference LayerOffload.store, sparse_offload.py:1131-1155). Row656 rows carry per-128
        scales of their own and kv_scale must be 1; Row400 rows quantize x / kv_scale (offload_rowfmt.store). Cached
        copies of the written rows are rewritten in HBM too (write-through), so both tiers hold the same values."""
        n = min(kv_c_normed.shape[0], slots.shape[0])
        if n == 0:
            return
        compact = self.row_fmt == "e2m2"
        if not compact and float(kv_scale) != 1.0:
            raise ValueError("LayerOffload.store: Row656 rows carry their own scales; kv_scale must be 1")
        kpe = k_pe.reshape(k_pe.shape[0], -1)
        slots = slots[:n].to(torch.int64)
        if self.trace is not None:
            self.trace.stored(slots)
        fmt = 2 if compact else 0
        kernels.cache_write(kv_c_normed[:n], kpe[:n], slots, self.host, fmt=fmt, kv_scale=kv_scale)
        if self.wc is not None:
            kernels.wcache_invalidate(self.wc, slots, self.R)      # rewritten rows: the next lookup misses
        elif self.C:
            ok = (slots >= 0) & (slots < self.R)
            lines = torch.where(ok, self.rowmap[slots.clamp(0, self.R - 1)].to(torch.int64), -1)
            if compact:
                # the cache lines get the compact rows (decoded for Row656 lines): encode the same tokens again into
                # HBM scratch (the encoder is deterministic) and copy or decode them into their lines
                tmp = self._buf("wt", (n, kernels.ROW400), torch.uint8)
                ident = torch.arange(n, dtype=torch.int64, device=self.device)
                kernels.cache_write(kv_c_normed[:n], kpe[:n], ident, tmp, fmt=2, kv_scale=kv_scale)
                if self.cache_fmt == "e2m2":
                    kernels.copy_rows(tmp, ident, self.cache[:self.C], lines)
                else:
                    kernels.row400_copy(tmp, ident, self.cache[:self.C], lines)
            else:
                kernels.cache_write(kv_c_normed[:n], kpe[:n], lines, self.cache[:self.C])

    def gather(self, rows, out):
        """out[i] = host row rows[i] (int64; zero row when outside [0, R)); out [N, 656] uint8 in HBM
        (reference LayerOffload.gather, sparse_offload.py:1157-1163). Compact host rows are decoded to out's
        format: [N, 656] Row656 or [N, 576] the reference's Row576 (offload_rowfmt.gather)."""
        if rows.shape[0]:
            if self.row_fmt == "e2m2":
                kernels.row400_gather(self.host, rows.to(torch.int64), out, pcie=True)
            else:
                kernels.gather(self.host, rows.to(torch.int64), out, pcie=True)
        return out

    def set_hot_rows(self, rows):
        """Make `rows` (distinct host rows, at most C) the HBM-resident set: line i holds rows[i]."""
        if self.wc is not None:
            raise ValueError("set_hot_rows: the W-way cache places rows itself (cache_mode='ways')")
        rows = rows.to(device=self.device, dtype=torch.int64).reshape(-1)
        if rows.numel() > self.C:
            raise ValueError(f"set_hot_rows: {rows.numel()} rows > {self.C} cache lines")
        old = self.tag[self.tag >= 0]
        if old.numel():
            self.rowmap[old] = -1
        self.tag.fill_(-1)
        m = rows.numel()
        if m:
            lines = torch.arange(m, dtype=torch.int64, device=self.device)
            if self.row_fmt == "e2m2" and self.cache_fmt != "e2m2":
                kernels.row400_copy(self.host, rows, self.cache[:self.C], lines)
            else:
                kernels.copy_rows(self.host, rows, self.cache[:self.C], lines)
            self.tag[:m] = rows
            self.rowmap[rows] = lines.to(torch.int32)

    # ------------------------------------------------------------------------------------------------ attention
    def _buf(self, name, shape, dtype):
        b = self._ws.get(name)
        n = 1
        for s in shape:
            n *= s
        if b is None or b.numel() < n or b.dtype != dtype:
            b = torch.empty(max(n, 1), dtype=dtype, device=self.device)
            self._ws[name] = b
        return b[:n].view(shape)

    def _attend_packed(self, q, idx, sm_scale, kv_scale, ql, out, lse, num_heads, return_lse):
        """Request-packed MTP decode: the union of each request's rows (mtp_union, rows once each with token masks),
        those rows staged in HBM -- hot rows copied from their cache lines, the others read over PCIe (decoded when the
        host rows are Row400) --, then one packed attention per request (attend_packed)."""
        T = q.shape[0]
        u, mk, cnt = kernels.mtp_union(idx, ql=ql, R=self.R)
        nreq, nmax = u.shape
        N = nreq * nmax
        uf = u.reshape(-1).to(torch.int64)
        pos = torch.arange(N, dtype=torch.int64, device=q.device)
        tiers = 2 if self.C else 1
        staged = self._buf("pk_staged", (tiers * N, ROW), torch.uint8)
        host_rows = uf
        if self.C:
            line = torch.where(uf >= 0, self.rowmap[uf.clamp(min=0)].to(torch.int64), torch.full_like(uf, -1))
            hit = line >= 0
            kernels.gather(self.cache, line, staged[:N])                    # hot rows from HBM (misses: zero rows)
            host_rows = torch.where(hit, torch.full_like(uf, -1), uf)
            su = torch.where(uf < 0, -1, torch.where(hit, pos, N + pos))
        else:
            su = torch.where(uf < 0, -1, pos)
        hs = staged[N * (tiers - 1):]
        if self.row_fmt == "e2m2":
            kernels.row400_gather(self.host, host_rows, hs, pcie=True)
        else:
            kernels.gather(self.host, host_rows, hs, pcie=True)
        su = su.to(torch.int32).view(nreq, nmax)
        kernels.attend_packed(q, staged, idx, sm_scale, kv_scale, ql=ql, out=out, lse=lse, union=(su, mk, cnt))
        return (out[:, :num_heads], lse[:, :num_heads]) if return_lse else out[:, :num_heads]

    def _side(self, device):
        """Second stream (default priority) and the two events that order it against the caller's stream."""
        if getattr(self, "_side_sync", None) is None:
            self._side_sync = (torch.cuda.Stream(device=device), torch.cuda.Event(), torch.cuda.Event())
        return self._side_sync

    def _identity(self, T, K, device):
        key = ("ident", T, K)
        b = self._ws.get(key)
        if b is None:
            b = torch.arange(T * K, dtype=torch.int32, device=device).view(T, K)
            self._ws[key] = b
        return b

    def attend(self, q, idx, sm_scale, kv_scale=1.0, num_heads=None, ql=1, mkey=None, slots=None, out=None,
               lse=None, return_lse=False):
        """q [T, H, 576] bf16, idx [T, K] int32 host rows (-1 / out of range = none) -> out [T, H, 512] bf16
        (reference LayerOffload.attend, sparse_offload.py:1350). return_lse: also the fp32 LSE [T, H]
        (ln sum exp of the scaled scores; -inf for a token without rows). ql: tokens per request; with packed=True and
        ql > 1 the request-packed path runs (same result up to the fp32 summation order); mkey / slots (the
        reference's prefetch hints) are accepted and do not change the result. With time_every set, the call is
        timed with GPU events (arm: packed / ways / tiers / host)."""
        if self.trace is not None:
            self.trace.access(idx, q.shape[0], self.C, self.W, self.R, slots)
        if self.stats_every:
            self._ncall += 1
            if self._ncall % self.stats_every == 0:
                self._stat(idx)
        e0 = self.timer.begin(q.device)
        res = self._attend(q, idx, sm_scale, kv_scale, num_heads, ql, out, lse, return_lse)
        if self.lstats_every and self.wc is not None:
            self._lcall += 1
            if self._lcall % self.lstats_every == 0:
                st = self.wc.state.tolist()
                self.log(f"[offl] L{self.layer} C={self.C} T={q.shape[0]} n={idx.numel()} hit={st[3]} miss={st[1]} "
                         f"spill={st[2]}")
        if e0 is not None:
            packed = self.packed and ql is not None and 1 < int(ql) <= 6 and q.shape[0] % int(ql) == 0
            arm = "packed" if packed else ("ways" if self.wc is not None else ("tiers" if self.C else "host"))
            self.timer.end(e0, arm, q.shape[0], q.device)
        return res

    def _attend(self, q, idx, sm_scale, kv_scale, num_heads, ql, out, lse, return_lse):
        T, H, _ = q.shape
        K = idx.shape[1]
        num_heads = H if num_heads is None else num_heads
        if out is None or out.shape != (T, H, kernels.D_LAT) or out.dtype != torch.bfloat16:
            out = torch.empty((T, H, kernels.D_LAT), dtype=torch.bfloat16, device=q.device)
        if lse is None:
            lse = torch.empty((T, H), dtype=torch.float32, device=q.device)
        if T == 0:
            return (out[:, :num_heads], lse[:, :num_heads]) if return_lse else out[:, :num_heads]
        if not torch.cuda.is_current_stream_capturing():    # the split merge's workspace, found by later captures
            kernels.reserve_workspace(q.device, H)
        idx = idx if idx.dtype == torch.int32 else idx.to(torch.int32)
        if self.packed and ql is not None and 1 < int(ql) <= 6 and T % int(ql) == 0:
            return self._attend_packed(q, idx, sm_scale, kv_scale, int(ql), out, lse, num_heads, return_lse)
        if self.wc is not None:
            return self._attend_ways(q, idx, sm_scale, kv_scale, out, lse, num_heads, return_lse)
        hbm = self._buf("hbm", (T, K), torch.int32)
        host = self._buf("host", (T, K), torch.int32)
        hcnt = self._buf("hcnt", (T,), torch.int32)
        mcnt = self._buf("mcnt", (T,), torch.int32)
        if self.C:
            kernels.tier_split(idx, self.rowmap, self.R, hbm, hcnt, host, mcnt)
        else:
            host = idx
            mcnt = None
        # host tier: copy the missed rows over PCIe into HBM staging, then attend there
        staged = self._buf("staged", (T * K, ROW), torch.uint8)
        compact = self.row_fmt == "e2m2"
        if not self.C:
            if compact:
                kernels.row400_gather(self.host, host.reshape(-1).to(torch.int64), staged, pcie=True)
            else:
                kernels.gather(self.host, host.reshape(-1).to(torch.int64), staged, pcie=True)
            sidx = self._buf("sidx", (T, K), torch.int32)
            ar = torch.arange(T * K, dtype=torch.int32, device=q.device).view(T, K)
            torch.where((host >= 0) & (host < self.R), ar, torch.full_like(ar, -1), out=sidx)
            kernels.attend(q, staged, sidx, sm_scale, kv_scale, out=out, lse=lse)
            return (out[:, :num_heads], lse[:, :num_heads]) if return_lse else out[:, :num_heads]
        if self.host_direct:
            return self._attend_host_direct(q, idx, sm_scale, kv_scale, out, lse, num_heads, return_lse, hbm, hcnt,
                                            host, mcnt)
        # the host list of token t is compacted (its mcnt[t] valid rows first): staged rows t * K + k, k < mcnt[t];
        # the attention's per-token count masks the rest, so the index map is the fixed identity
        sidx = self._identity(T, K, q.device)
        op = self._buf("opart", (1, T, H, kernels.D_LAT), torch.float32)
        lp = self._buf("lpart", (1, T, H), torch.float32)
        # the PCIe copy (64 workgroups) runs beside the HBM-tier attention, which is queued on a second stream of
        # default priority; the host-tier attention waits for it and merges its partial in its own epilogue
        main = torch.cuda.current_stream(q.device)
        side, ev_split, ev_hbm = self._side(q.device)
        ev_split.record(main)
        if compact:
            kernels.row400_gather_tiers(self.host, host, mcnt, staged)
        else:
            kernels.gather_tiers(self.host, host, mcnt, staged)
        side.wait_event(ev_split)
        with torch.cuda.stream(side):
            if self.cache_fmt == "e2m2":
                # compact lines: decode the step's hot lines (compacted per token, -1 padded) into Row576 staging in
                # the same order (the decoded values are Row576 values), then attend there through the identity map
                hstaged = self._buf("hstaged", (T * K, kernels.ROW576), torch.uint8)
                kernels.row400_decode_tiers(self.cache[:self.C], hbm, hcnt, hstaged)
                kernels.attend_partial(q, hstaged, sidx, sm_scale, kv_scale, op[0:1], lp[0:1], kcount=hcnt)
            else:
                kernels.attend_partial(q, self.cache[:self.C], hbm, sm_scale, kv_scale, op[0:1], lp[0:1],
                                       kcount=hcnt)
            ev_hbm.record(side)
        main.wait_event(ev_hbm)
        kernels.attend_merge(q, staged, sidx, sm_scale, kv_scale, op[0], lp[0], out=out, lse=lse, kcount=mcnt)
        return (out[:, :num_heads], lse[:, :num_heads]) if return_lse else out[:, :num_heads]

    def _attend_host_direct(self, q, idx, sm_scale, kv_scale, out, lse, num_heads, return_lse, hbm, hcnt, host, mcnt):
        """Two tiers, no staging copy: the HBM-tier attention (second stream) runs beside an attention that reads
        each token's host rows in place from the pinned pool over PCIe; the two partials are then merged."""
        T, H, _ = q.shape
        op = self._buf("opart2", (2, T, H, kernels.D_LAT), torch.float32)
        lp = self._buf("lpart2", (2, T, H), torch.float32)
        main = torch.cuda.current_stream(q.device)
        side, ev_split, ev_hbm = self._side(q.device)
        ev_split.record(main)
        side.wait_event(ev_split)
        with torch.cuda.stream(side):
            kernels.attend_partial(q, self.cache[:self.C], hbm, sm_scale, kv_scale, op[0:1], lp[0:1], kcount=hcnt)
            ev_hbm.record(side)
        kernels.attend_partial(q, self.host, host, sm_scale, kv_scale, op[1:2], lp[1:2], kcount=mcnt, R=self.R)
        main.wait_event(ev_hbm)
        kernels.lse_merge(op, lp, out=out, lse=lse)
        return (out[:, :num_heads], lse[:, :num_heads]) if return_lse else out[:, :num_heads]

    def _attend_ways(self, q, idx, sm_scale, kv_scale, out, lse, num_heads, return_lse):
        """W-way cache step: look up / place / resolve, copy the misses in, attend over the pool. Entries left on
        the host (spill area full) take the host tier, merged in the host-tier attention's epilogue. Compact Row400
        lines (cache_fmt="e2m2") are decoded per step into staging in the order of the row list the attention
        reads (Row576 staging for the hits, Row656 for the fresh rows that take the merging attention)."""
        T, H, _ = q.shape
        K = idx.shape[1]
        wc = self.wc
        compact_pool = self.cache_fmt == "e2m2"
        res = self._buf("res", (T, K), torch.int32)
        fmt = 2 if self.row_fmt == "e2m2" else 0
        ident = self._identity(T, K, q.device)

        def pool_rows(rows, name, width, counts=None):
            """(pool, index map) the attention reads for pool rows `rows` [T, K] (< 0: none): the pool itself, or the
            rows decoded into staging row t * K + k -- for lists compacted per token (counts: the attention reads
            only those entries) the identity map, else a map that keeps the entries without a row at -1."""
            if not compact_pool:
                return wc.pool, rows
            st = self._buf(name, (T * K, width), torch.uint8)
            kernels.row400_decode_tiers(wc.pool, rows, counts, st)
            if counts is not None:
                return st, ident
            m = self._buf(name + "_map", (T, K), torch.int32)
            torch.where(rows >= 0, ident, torch.full_like(ident, -1), out=m)
            return st, m

        if T * K <= wc.cap and self.overlap_fill:
            # placement, then the PCIe copy of the misses on the second stream while the resolution, the hit / fresh
            # split and the attention over the hits run here; the fresh rows' attention merges the hits' partial
            kernels.wcache_place(wc, idx, self.R)
            main = torch.cuda.current_stream(q.device)
            side, ev_place, ev_fill = self._side(q.device)
            ev_place.record(main)
            side.wait_event(ev_place)
            with torch.cuda.stream(side):
                kernels.wcache_fill(wc, self.host, self.R, fmt, T * K)
                ev_fill.record(side)
            kernels.wcache_resolve(wc, idx, self.R, res)
            hit = self._buf("hbm", (T, K), torch.int32)
            fresh = self._buf("host", (T, K), torch.int32)
            hcnt = self._buf("hcnt", (T,), torch.int32)
            fcnt = self._buf("mcnt", (T,), torch.int32)
            kernels.wcache_split(wc, res, hit, hcnt, fresh, fcnt)
            op = self._buf("opart", (1, T, H, kernels.D_LAT), torch.float32)
            lp = self._buf("lpart", (1, T, H), torch.float32)
            src, rows = pool_rows(hit, "hstaged", kernels.ROW576, hcnt)
            kernels.attend_partial(q, src, rows, sm_scale, kv_scale, op, lp, kcount=hcnt)
            main.wait_event(ev_fill)
            src, rows = pool_rows(fresh, "fstaged", ROW, fcnt)
            kernels.attend_merge(q, src, rows, sm_scale, kv_scale, op[0], lp[0], out=out, lse=lse, kcount=fcnt)
            return (out[:, :num_heads], lse[:, :num_heads]) if return_lse else out[:, :num_heads]
        kernels.wcache_step(wc, idx, self.R, res)
        kernels.wcache_fill(wc, self.host, self.R, fmt, T * K)
        if T * K <= wc.cap:                                  # every miss fits the spill area: one HBM tier
            src, rows = pool_rows(res, "hstaged", kernels.ROW576)
            kernels.attend(q, src, rows, sm_scale, kv_scale, out=out, lse=lse)
        else:
            hbm = self._buf("hbm", (T, K), torch.int32)
            host = self._buf("host", (T, K), torch.int32)
            hcnt = self._buf("hcnt", (T,), torch.int32)
            mcnt = self._buf("mcnt", (T,), torch.int32)
            kernels.split_res(idx, res, hbm, hcnt, host, mcnt)
            op = self._buf("opart", (1, T, H, kernels.D_LAT), torch.float32)
            lp = self._buf("lpart", (1, T, H), torch.float32)
            src, rows = pool_rows(hbm, "hstaged", kernels.ROW576, hcnt)
            kernels.attend_partial(q, src, rows, sm_scale, kv_scale, op, lp, kcount=hcnt)
            staged = self._buf("staged", (T * K, ROW), torch.uint8)
            if self.row_fmt == "e2m2":
                kernels.row400_gather_tiers(self.host, host, mcnt, staged)
            else:
                kernels.gather_tiers(self.host, host, mcnt, staged)
            kernels.attend_merge(q, staged, ident, sm_scale, kv_scale, op[0], lp[0], out=out, lse=lse, kcount=mcnt)
        return (out[:, :num_heads], lse[:, :num_heads]) if return_lse else out[:, :num_heads]

    def _stat(self, idx):
        f = idx.reshape(-1).to(torch.int64)
        f = f[(f >= 0) & (f < self.R)]
        if f.numel():
            self.log(f"[offstats] C={self.C} rows={f.numel()} uniq={int(torch.unique(f).numel())} "
                     f"hit={self.hit_rate(f.reshape(1, -1)):.3f}")

    def hit_rate(self, idx):
        """Fraction of the valid selected rows of idx [T, K] that the HBM cache holds."""
        v = (idx >= 0) & (idx < self.R)
        if self.wc is not None:
            f = idx.reshape(-1).to(torch.int64)
            f = f[(f >= 0) & (f < self.R)]
            return float(self.wc.lookup(f).float().mean()) if f.numel() else 0.0
        if not self.C or not bool(v.any()):
            return 0.0
        hit = self.rowmap[idx.clamp(0, self.R - 1).long()] >= 0
        return float((hit & v).sum()) / float(v.sum())
