"""Serving-time diagnostics of the path, off by default, as the reference has them:

- AttnTimer: GPU events around every decode attention call, read back 64 calls later (no synchronization in the
  serving loop), mean ms per call per arm printed every N calls (the reference's ARC_OFFLOAD_ATTN2_TIME ring,
  dotsnote/engine/arcstats_pkg/arcstats/offload_cuda2.py:135-170).
- verify_outputs: the offload path's output against the paged path's on the same step, per token, with the bad
  tokens reported (ARC_OFFLOAD_VERIFY, dotsnote/engine/arcstats_pkg/arcstats/dsa_sm89.py:396-424).
- TopkCheck: recall of the kernel's top-k rows against torch.topk over the same logits (ARC_SHARD_CHECK,
  dotsnote/engine/arcstats_pkg/arcstats/shard_indexer.py:224-279, which re-derives the logits from a replicated key
  store; on one GPU the store is already whole, so the check is of the selection).
- AccessTrace: a layer's stored slots and decode top-k rows over a window of calls, saved to an .npz for offline
  row-cache simulation (ARC_OFFLOAD_DUMP / ARC_OFFLOAD_DUMP_LAYERS,
  dotsnote/engine/arcstats_pkg/arcstats/sparse_offload.py:33-35, :1063-1071, :1516-1538).
"""
import os
import re
import time

import numpy as np
import torch


class AttnTimer:
    """Event pairs per call; a pair is read once 128 are queued (the oldest 64, long finished), so the serving loop
    never waits. stats[arm] = [calls, total ms, total tokens]."""

    def __init__(self, every, log=print):
        self.every = int(every)
        self.log = log
        self.queue = []
        self.stats = {}

    def begin(self, device):
        if not self.every:
            return None
        e = torch.cuda.Event(enable_timing=True)
        e.record(torch.cuda.current_stream(device))
        return e

    def end(self, e0, arm, T, device):
        if e0 is None:
            return
        e1 = torch.cuda.Event(enable_timing=True)
        e1.record(torch.cuda.current_stream(device))
        self.queue.append((arm, int(T), e0, e1))
        if len(self.queue) >= 128:
            self.drain(64)

    def drain(self, n=None):
        """Read the oldest n pairs (all when None) into the statistics; print a line every `every` calls."""
        n = len(self.queue) if n is None else n
        before = sum(v[0] for v in self.stats.values())
        for arm, T, a, b in self.queue[:n]:
            b.synchronize()
            s = self.stats.setdefault(arm, [0, 0.0, 0])
            s[0] += 1
            s[1] += a.elapsed_time(b)
            s[2] += T
        del self.queue[:n]
        after = sum(v[0] for v in self.stats.values())
        if self.every and after // self.every != before // self.every:
            self.log("[attn time] " + "  ".join(
                f"{k}: n={v[0]} {v[1] / v[0]:.3f} ms/call T={v[2] / v[0]:.0f} {256 * v[1] / max(v[2], 1):.3f} ms/256tok"
                for k, v in sorted(self.stats.items())))
        return self.stats


def verify_outputs(o_test, o_ref, stats, label="", tol=0.1, log=print):
    """Per token t: rel[t] = max |o_test - o_ref| / max(max |o_ref|, 1e-3) over heads and dims; tokens with rel > tol
    are reported (at most 400 reports). stats (a dict) accumulates calls, tokens, bad tokens and the largest rel.
    Returns rel [T] (float32, on o_ref's device)."""
    d = (o_test.float() - o_ref.float()).abs().amax(dim=(1, 2))
    ref = o_ref.float().abs().amax(dim=(1, 2)).clamp_min(1e-3)
    rel = d / ref
    bad = (rel > tol).nonzero().flatten()
    stats["calls"] = stats.get("calls", 0) + 1
    stats["tokens"] = stats.get("tokens", 0) + int(rel.numel())
    stats["bad"] = stats.get("bad", 0) + int(bad.numel())
    stats["max_rel"] = max(stats.get("max_rel", 0.0), float(rel.max()) if rel.numel() else 0.0)
    if bad.numel() and stats.get("reports", 0) < 400:
        stats["reports"] = stats.get("reports", 0) + 1
        log(f"[verify] {label} call={stats['calls']} tokens={rel.numel()} bad={bad.numel()} "
            f"first={bad[:8].tolist()} rel.max={float(rel.max()):.3f}")
    return rel


class TopkCheck:
    """Recall of selected rows against torch.topk on the same logits: per row |ref ∩ got| / |ref| over the
    non-negative entries (ref = torch.topk of the row's first ctx columns, +-inf values dropped)."""

    def __init__(self, every=2000, log=print):
        self.every = int(every)
        self.log = log
        self.rows = 0
        self.recall = 0.0
        self.min_recall = 1.0

    def check(self, lg, ctx, got, kk):
        n = lg.shape[0]
        for r in range(n):
            c = max(0, min(int(ctx[r]), lg.shape[1]))
            k = min(kk, c)
            a = set()
            if k:
                v, j = torch.topk(lg[r, :c].float(), k)
                a = set(j[torch.isfinite(v)].tolist())
            g = got[r]
            b = set(g[g >= 0].tolist())
            rec = len(a & b) / max(1, len(a))
            self.rows += 1
            self.recall += rec
            self.min_recall = min(self.min_recall, rec)
        if self.every and self.rows % self.every < n:
            self.log(f"[shardcheck] rows={self.rows} mean recall={self.recall / self.rows:.5f} "
                     f"min={self.min_recall:.4f}")
        return self.recall / max(1, self.rows)


class AccessTrace:
    """Events of one offload layer for offline row-cache simulation (reference LayerOffload._record,
    sparse_offload.py:1516-1538). Recording starts at the first attend call with T >= min_t once after_s seconds
    have passed; from then on each store() appends its slots (kind 0) and each attend call its rows (kind 1): the
    distinct valid rows sorted (unique=True, the reference's per-layer dump, which also takes the step's slots passed
    to attend as a kind-0 event first) or the whole int32 idx [T, K] (unique=False). After `calls` attend calls the
    events go to `path`.npz with np.savez_compressed: kinds int8 [E], C, W, R, T (the last call's tokens) and e0 ..
    e{E-1}, the same keys as the reference's file. Each recorded call reads its rows back to the host (a
    synchronization): a diagnostic, off by default."""

    def __init__(self, path, calls, after_s=0.0, min_t=1, unique=False, clock=time.time, log=print):
        if int(calls) <= 0:
            raise ValueError("AccessTrace: calls must be positive")
        self.path = str(path)
        self.left = int(calls)
        self.t0 = clock() + float(after_s)
        self.min_t = int(min_t)
        self.unique = bool(unique)
        self.clock = clock
        self.log = log
        self.on = False
        self.done = False
        self.events = []

    @classmethod
    def from_env(cls, key=None, device=None, first=True, env=None, **kw):
        """The reference's switches: ARC_OFFLOAD_DUMP=path,after_s,calls,min_T names the file and window;
        ARC_OFFLOAD_DUMP_LAYERS=1,17,... picks backbone layers by the number in `key` (its 'layers.<n>.' part), each
        to path_L<n>.npz with unique rows, else the first offload layer (first=True) dumps to path.npz with whole
        idx arrays. Only device index 0 (or a device without index) records. None when nothing applies."""
        env = os.environ if env is None else env
        spec = env.get("ARC_OFFLOAD_DUMP", "")
        if not spec:
            return None
        if device is not None and torch.device(device).index not in (0, None):
            return None
        m = re.search(r"layers\.(\d+)\.", key or "")
        layer = int(m.group(1)) if m else -1
        dl = env.get("ARC_OFFLOAD_DUMP_LAYERS", "")
        if dl:
            if layer not in {int(x) for x in dl.split(",") if x}:
                return None
        elif not first:
            return None
        path, after, calls, min_t = spec.split(",")
        return cls(path + (f"_L{layer}" if dl else ""), int(calls), float(after), int(min_t), unique=bool(dl), **kw)

    def stored(self, slots):
        """store() of n slots: a kind-0 event while recording."""
        if self.on and not self.done:
            self.events.append((0, slots.to(torch.int32).cpu().numpy()))

    def access(self, idx, T, C, W, R, slots=None):
        """attend() over idx [T, K] (-1 = none): a kind-1 event (and the slots' kind-0 event in unique mode);
        writes the file when the window is full."""
        if self.done:
            return
        if not self.on:
            if int(T) < self.min_t or self.clock() < self.t0:
                return
            self.on = True
            self.log(f"[offdump] start T={int(T)} C={C} W={W} R={R}")
        if self.unique:
            if slots is not None:
                self.events.append((0, slots.to(torch.int32).cpu().numpy()))
            f = idx.reshape(-1)
            self.events.append((1, torch.unique(f[f >= 0]).to(torch.int32).cpu().numpy()))
        else:
            self.events.append((1, idx.to(torch.int32).cpu().numpy()))
        self.left -= 1
        if self.left <= 0:
            kinds = np.array([k for k, _ in self.events], dtype=np.int8)
            np.savez_compressed(self.path, kinds=kinds, C=int(C), W=int(W), R=int(R), T=int(T),
                                **{f"e{i}": a for i, (_, a) in enumerate(self.events)})
            self.log(f"[offdump] saved {len(self.events)} events to {self.path}.npz")
            self.done = True
            self.events = []
