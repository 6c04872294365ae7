"""Serving-time diagnostics of the path, off by default, as the reference has them:

- AttnTimer: GPU events around every decode attention call, read back 64 calls later (no synchronization in the
  serving loop), mean ms per call per arm printed every N calls (the reference's ARC_OFFLOAD_ATTN2_TIME ring,
  dotsnote/engine/arcstats_pkg/arcstats/offload_cuda2.py:135-170).
- verify_outputs: the offload path's output against the paged path's on the same step, per token, with the bad
  tokens reported (ARC_OFFLOAD_VERIFY, dotsnote/engine/arcstats_pkg/arcstats/dsa_sm89.py:396-424).
- TopkCheck: recall of the kernel's top-k rows against torch.topk over the same logits (ARC_SHARD_CHECK,
  dotsnote/engine/arcstats_pkg/arcstats/shard_indexer.py:224-279, which re-derives the logits from a replicated key
  store; on one GPU the store is already whole, so the check is of the selection).
"""
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
