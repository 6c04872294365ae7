"""Benchmark of the MI355X sparse-MLA decode path (BASELINE.json metric: "sparse-MLA decode step us + effective GB/s
(% of 8 TB/s), B=64 ctx32K top2048").

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--config 1|2|3|4|5] [--no-variant]

Default (--config 2) = BASELINE config 2, all-HBM decode: B = 64 sequences, 128 query heads, 32768-token context per
sequence held as Row656 KV rows in HBM (latent / rope N(0,1), written by the library's own cache-write kernel), q bf16
N(0,1), top-2048 row indices per sequence drawn uniformly without replacement, softmax scale 1/sqrt(192), bf16 out +
fp32 LSE. One step = one spmla_attn_splitk launch over the whole batch (inputs resident in HBM). `value` = effective
GB/s = algorithmic bytes / step time, algorithmic bytes = 131072 rows x 656 B + q + idx + out + lse = 104,366,080 B.
`roofline` is timed live with HIP events on the stream the kernel is launched on, and its `traffic` (HBM bytes per
launch) is counted in the same run: four rocprofv3 --pmc child runs (FETCH_SIZE and WRITE_SIZE over a few probe
launches, and over a plain 256 MiB device copy that calibrates the counters; --no-traffic skips them); `cpu_baseline` times the float32
torch-CPU restatement (oracle/cpu_port.py) of the same step on this host's cores. Unless --no-variant, the line also
carries `host_tier_variant`: BASELINE config 3 (same shapes, 2M-row pool in pinned host memory, 25% HBM hot set,
Zipf(1.1) selections) measured in the same run, and `host_tier_compact_variant`: the same with the host pool in the
reference's compact Row400 rows (decoded on the way in; 400 instead of 656 bytes per row over PCIe), and
`host_tier_compact_cache_variant` keeps the static hot set as compact Row400 lines in HBM (`--host-rows e2m2
--cache-fmt e2m2`); `host_tier_production_variant` is the reference's shipped offload mode (mode_submit.json: compact
host rows, a dynamic 8-way two-choice row cache of compact Row400 lines, the miss copy beside the attention over the
hits) on a stream of fresh Zipf draws (`--config 3 --cache ways --ways 8 --two-choice --host-rows e2m2 --cache-fmt
e2m2`); `host_tier_overflow_one_choice_variant` / `..._two_choice_variant` run it with a 131,072-line cache (the
reference's two-choice geometry, offload_fill.py:16-20), whose sets overflow, without and with two-choice placement,
reporting misses and spill rows per step.

Other configs print their own JSON line (same keys): 1 = B=1 / 16 heads / K=256 check + timing, 3 = offload split-K,
4 = indexer logits + top-2048 at L = 32768 and 131072, 5 = chunked prefill (8192 queries) + cache write, 6 = the
absorbed FP8 matmuls either side of the decode attention (query build + output).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

B, H, CTX, K, D = 64, 128, 32768, 2048, 576
ROWB = 656
SM_SCALE = 192 ** -0.5
ALG_BYTES = B * K * ROWB + B * H * D * 2 + B * K * 4 + B * H * 512 * 2 + B * H * 4
ALG_FLOPS = B * H * K * (2 * 576 + 2 * 512)
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
METRIC = "sparse-MLA decode step us + effective GB/s (% of 8 TB/s), B=64 ctx32K top2048"


# ------------------------------------------------------------------------------------------------ helpers
def _timed(fn, steps, warmup):
    """Average ms of fn() over `steps` calls (after `warmup`), HIP events on the current stream (the stream every
    library entry point launches on)."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(steps):
        fn()
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def _settle(fn, seconds=0.2):
    """fn() back to back for `seconds` of wall time, untimed, before a timed region. The GPU's clocks ramp under
    sustained load: the config-2 decode kernel takes ~75 us per launch in its first 100 launches, ~59.5 us from
    ~800 launches (~50 ms) on, and ~66 us again after a second of idling. A decode server runs in that steady
    state, so the timed steps start there."""
    import torch
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(4):
            fn()
        torch.cuda.synchronize()


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo, as lscpu prints it) and its logical CPU count."""
    name, n = None, 0
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    n += 1
                    name = name or line.split(":", 1)[1].strip()
    except OSError:
        pass
    return f"{name or 'unknown'} ({n} logical CPUs)" if n else (name or "unknown")


def _with_model(cpu):
    if isinstance(cpu, dict) and "cpu_model" not in cpu:
        cpu = dict(cpu, cpu_model=cpu_model())
    return cpu


def _line(metric, value, unit, a, ms, dtype, config, roofline, cpu=None, hib=True, **extra):
    res = {"metric": metric, "value": round(value, 3), "unit": unit, "n_gpus": 1, "steps": a.steps,
           "warmup": a.warmup, "ms_per_step": round(ms, 5), "higher_is_better": hib, "scaling": "weak",
           "vs_baseline": None, "dtype": dtype, "data": "synthetic (seeded)", "config": config,
           "roofline": roofline, "cpu_baseline": _with_model(cpu)}
    res.update(extra)
    return res


def _cache_fill(pool_u8, nrows, seed, dev, fmt=0):
    """Rows 0..nrows of pool_u8 (device or pinned host) written from seeded N(0,1) bf16 latents / ropes by the
    library's cache-write kernel (fmt 0 = Row656, 1 = Row576 and 2 = compact Row400, both with kv_scale 1)."""
    import torch
    from arcagi2_flashnext_dots3_amd import kernels
    g = torch.Generator(device=dev).manual_seed(seed)
    chunk = 1 << 18
    for r0 in range(0, nrows, chunk):
        n = min(chunk, nrows - r0)
        kv = torch.randn(n, 512, generator=g, device=dev).to(torch.bfloat16)
        pe = torch.randn(n, 64, generator=g, device=dev).to(torch.bfloat16)
        slots = torch.arange(r0, r0 + n, dtype=torch.int64, device=dev)
        kernels.cache_write(kv, pe, slots, pool_u8, fmt=fmt)
    torch.cuda.synchronize()


# ------------------------------------------------------------------------------------------------ config 2
def build_inputs(dev, nsets=1):
    import torch
    R = B * CTX
    pool = torch.empty(R, ROWB, dtype=torch.uint8, device=dev)
    _cache_fill(pool, R, 1, dev)
    gq = torch.Generator().manual_seed(0)
    q = torch.randn(B, H, D, generator=gq).to(torch.bfloat16).to(dev)
    idxs = []
    for n in range(nsets):
        gi = torch.Generator().manual_seed(2 + n)
        idxs.append(torch.stack([torch.randperm(CTX, generator=gi)[:K] + b * CTX for b in range(B)])
                    .to(torch.int32).to(dev))
    torch.cuda.synchronize()
    return pool, q, idxs


def cpu_baseline(pool, q, idx):
    import torch
    from oracle import cpu_port
    nt = cpu_port.threads()
    torch.set_num_threads(nt)
    # bounded sample: the rows this step selects (the whole step's inputs), on the host
    flat = idx.reshape(-1).long()
    rows_host = pool[flat].cpu()                                  # [B*K, 656]
    idx_local = torch.arange(B * K, dtype=torch.int32).reshape(B, K)
    qh = q.cpu()
    cpu_port.attention_f32(qh, rows_host, idx_local, SM_SCALE)    # warm-up
    ts = []
    for _ in range(5):
        t0 = time.perf_counter()
        cpu_port.attention_f32(qh, rows_host, idx_local, SM_SCALE)
        ts.append(time.perf_counter() - t0)
    ts.sort()
    t = ts[2]
    return {"value": round(ALG_BYTES / t / 1e9, 3), "unit": "GB/s", "cores": nt, "kind": "port",
            "sample": f"full config-2 step (B=64, H=128, K=2048) in fp32 torch on {nt} threads, median of 5: "
                      f"{t * 1e3:.1f} ms/step"}


def run_config2(a, dev):
    """BASELINE config 2. The step is one attention launch over one of `idx_sets` selections (rotating). Timed as a
    decode loop runs it, from a HIP graph that holds one launch per selection set and is replayed; the eager loop
    (host dispatch from Python included) is timed beside it."""
    import torch
    from arcagi2_flashnext_dots3_amd import kernels
    pool, q, idxs = build_inputs(dev, a.idx_sets)
    out = torch.empty(B, H, 512, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(B, H, dtype=torch.float32, device=dev)
    split = kernels.auto_split(B, H, K)
    # the split merge's workspace, zeroed once here: one allocated inside the graph capture would be zero-filled by
    # every replay (the kernel leaves its counters at zero, so it needs that only once)
    ws = torch.zeros(max(1, int(kernels.attn_ws_bytes(B, H, split))), dtype=torch.uint8, device=dev)
    cur = [0]

    def launch(i):
        kernels.attend(q, pool, idxs[i], SM_SCALE, out=out, lse=lse, split=split, ws=ws)

    def step():
        launch(cur[0] % len(idxs))
        cur[0] += 1

    n = len(idxs)
    replay = _graphed(lambda: [launch(i) for i in range(n)], 1)
    reps = max(1, a.steps // n)
    _settle(replay)
    ms = _timed(replay, reps, max(1, a.warmup // n)) / n
    eager_ms = _timed(step, a.steps, a.warmup)          # right after, at the same settled clocks
    gbs = ALG_BYTES / (ms * 1e-3) / 1e9
    # unsplit decode launches run the head-group kernel, split ones the 128-head kernel with its in-kernel merge
    kname = "spmla::pk::attn_kernel<false, false>" if split == 1 else "spmla::attn::fwd_kernel"
    roof = {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": kname, "alg_bytes_per_launch": ALG_BYTES,
            "mfma_tflops": round(ALG_FLOPS / (ms * 1e-3) / 1e12, 2),
            "mfma_frac_bf16_peak": round(ALG_FLOPS / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4)}
    if not a.no_traffic:     # HBM bytes per launch, counted in this run (rocprofv3 --pmc over probe children)
        tr = measure_traffic(r"attn_kernel<false, false>" if split == 1 else "fwd_kernel",
                             ["--config", "2", "--probe", "--idx-sets", str(a.idx_sets)])
        roof["traffic"] = tr.get("bytes_per_launch")
        roof["traffic_detail"] = tr
    cfg = {"workload": "BASELINE config 2: all-HBM sparse-MLA decode, B=64, H=128, ctx=32768/seq, top-2048, Row656 "
                       "rows, bf16 out + fp32 LSE; launches replayed from a HIP graph after 0.2 s of untimed back-to-back "
                       "launches (steady-state clocks)",
           "global_batch": B, "heads": H, "ctx": CTX, "topk": K, "row_bytes": ROWB, "idx_sets": a.idx_sets}
    res = _line(METRIC, gbs, "GB/s", a, ms, "fp8e4m3 rows x bf16 q: bf16 MFMA (QK), f16 MFMA (PV), fp32 accumulate",
                cfg, roof, step_us=round(ms * 1e3, 2), eager_step_us=round(eager_ms * 1e3, 2))
    if not a.no_cpu:
        res["cpu_baseline"] = _with_model(cpu_baseline(pool, q, idxs[0]))
    del pool
    torch.cuda.empty_cache()
    if not a.no_variant:
        res["row576_variant"] = run_row576(a, dev, q, idxs, out, lse)
    return res


def run_probe(a, dev):
    """A few eager launches of config 2's step and nothing else (the launches a counter run reads)."""
    import torch
    from arcagi2_flashnext_dots3_amd import kernels
    pool, q, idxs = build_inputs(dev, a.idx_sets)
    out = torch.empty(B, H, 512, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(B, H, dtype=torch.float32, device=dev)
    for i in range(2 * len(idxs)):
        kernels.attend(q, pool, idxs[i % len(idxs)], SM_SCALE, out=out, lse=lse)
    torch.cuda.synchronize()
    return {"probe_launches": 2 * len(idxs)}


def _pmc(counter, regex, args, timeout=180):
    """Average per-dispatch value of one rocprofv3 counter over the kernels matching regex, in a child run of this
    script with `args` (from /tmp, as rocprofv3 wants); None when the profiler or the child fails."""
    import csv
    import re
    import subprocess
    import tempfile
    d = tempfile.mkdtemp(prefix="spmla_pmc_", dir="/tmp")
    cmd = ["rocprofv3", "--pmc", counter, "--output-format", "csv", "-d", d, "-o", "run", "--",
           sys.executable, os.path.abspath(__file__)] + args
    env = dict(os.environ, TMPDIR="/tmp")
    try:
        subprocess.run(cmd, cwd="/tmp", env=env, capture_output=True, timeout=timeout)
    except Exception:
        return None
    vals = []
    for root, _, files in os.walk(d):
        for f in files:
            if f.endswith("counter_collection.csv"):
                for row in csv.DictReader(open(os.path.join(root, f))):
                    if row.get("Counter_Name") == counter and re.search(regex, row.get("Kernel_Name", "")):
                        vals.append(float(row["Counter_Value"]))
    return sum(vals) / len(vals) if vals else None


def measure_traffic(regex, args, calib=1 << 28):
    """HBM bytes per launch of the kernels matching regex: FETCH_SIZE and WRITE_SIZE (KiB per dispatch) each scaled
    by the bytes a plain device copy of `calib` bytes moves per KiB that counter reads for it, four counter runs of
    child processes in this run (one counter per run)."""
    fk = _pmc("FETCH_SIZE", regex, args)
    wk = _pmc("WRITE_SIZE", regex, args)
    cf = _pmc("FETCH_SIZE", "copyBuffer", ["--copy-calib", str(calib)])
    cw = _pmc("WRITE_SIZE", "copyBuffer", ["--copy-calib", str(calib)])
    if None in (fk, wk, cf, cw) or cf <= 0 or cw <= 0:
        return {"bytes_per_launch": None, "error": "a counter run failed",
                "fetch_kib": fk, "write_kib": wk, "copy_fetch_kib": cf, "copy_write_kib": cw}
    ff, fw = calib / (cf * 1024), calib / (cw * 1024)
    return {"bytes_per_launch": int(round(fk * 1024 * ff + wk * 1024 * fw)), "fetch_kib": round(fk, 1),
            "write_kib": round(wk, 1), "fetch_factor": round(ff, 4), "write_factor": round(fw, 4),
            "source": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE in this run, scaled by a plain copy's readings"}


def run_row576(a, dev, q, idxs, out, lse):
    """Config 2's step over the plugin's per-tensor fp8 cache (Row576 rows: 512 + 64 e4m3 codes, kv_scale 1, written
    by the library from the same seeded latents), attended in place by spmla_attn576; timed like the main line."""
    import torch
    from arcagi2_flashnext_dots3_amd import kernels
    R = B * CTX
    pool = torch.empty(R, 576, dtype=torch.uint8, device=dev)
    _cache_fill(pool, R, 1, dev, fmt=1)
    n = len(idxs)
    replay = _graphed(lambda: [kernels.attend(q, pool, idxs[i], SM_SCALE, out=out, lse=lse, split=1)
                               for i in range(n)], 1)
    _settle(replay)
    ms = _timed(replay, max(1, a.steps // n), max(1, a.warmup // n)) / n
    alg = ALG_BYTES - B * K * (ROWB - 576)
    gbs = alg / (ms * 1e-3) / 1e9
    del pool
    torch.cuda.empty_cache()
    return {"step_us": round(ms * 1e3, 2), "gbs": round(gbs, 2), "frac": round(gbs / HBM_PEAK_GBS, 4),
            "alg_bytes_per_launch": alg, "kernel": "spmla::pk::attn_kernel<false, true>",
            "mfma_tflops": round(ALG_FLOPS / (ms * 1e-3) / 1e12, 2),
            "workload": "config 2 (B=64, H=128, top-2048 of 32768 rows per sequence) over Row576 rows (the plugin's "
                        "fp8 cache: 576 B/row, per-tensor scale), one launch per step from a HIP graph"}


# ------------------------------------------------------------------------------------------------ config 3
R3 = 2097152


def zipf_selections(nseq, K, R, seed, s=1.1, perm=None, device="cpu"):
    """Per sequence K distinct rows: Zipf(s) ranks (P(r) ~ r^-s over R ranks) mapped through a seeded permutation of
    the pool, repeated draws rejected (first appearances kept in draw order). Returns int64 [nseq, K] on `device`."""
    import torch
    if perm is None:
        perm = torch.randperm(R, generator=torch.Generator().manual_seed(3))
    perm = perm.to(device)
    cdf = torch.cumsum(torch.arange(1, R + 1, dtype=torch.float64, device=device) ** (-s), 0)
    cdf /= cdf[-1].clone()
    g = torch.Generator(device=device).manual_seed(seed)
    M = 6 * K
    out = torch.empty((nseq, K), dtype=torch.int64, device=device)
    for b0 in range(0, nseq, 256):
        n = min(256, nseq - b0)
        r = torch.searchsorted(cdf, torch.rand(n, M, generator=g, device=device, dtype=torch.float64))
        r = r.clamp_(max=R - 1)
        rs, order = torch.sort(r, dim=1, stable=True)                # equal ranks keep draw order
        first = torch.ones_like(rs, dtype=torch.bool)
        first[:, 1:] = rs[:, 1:] != rs[:, :-1]
        pos = torch.sort(torch.where(first, order, torch.full_like(order, M)), dim=1).values[:, :K]
        if bool((pos[:, -1] >= M).any()):
            raise RuntimeError("zipf_selections: too few distinct draws; raise M")
        out[b0:b0 + n] = perm[torch.gather(r, 1, pos)]
    return out


def run_config3(a, dev, steps=None, row_fmt="row656", cache_fmt="row656", host_direct=False):
    import torch
    from arcagi2_flashnext_dots3_amd import kernels
    from arcagi2_flashnext_dots3_amd.sparse_offload import HOST_ROW, LayerOffload, hot_rows_by_frequency
    steps = steps or a.steps
    C = R3 // 4
    compact = row_fmt == "e2m2"
    lo = LayerOffload(R3, dev, cache_rows=C, row_fmt=row_fmt, cache_fmt=cache_fmt, host_direct=host_direct)
    _cache_fill(lo.host, R3, 1, dev, fmt=2 if compact else 0)
    perm = torch.randperm(R3, generator=torch.Generator().manual_seed(3))
    warm = zipf_selections(64 * B, K, R3, seed=4, perm=perm, device=dev)   # 64 warm-up steps of B sequences
    counts = torch.bincount(warm.reshape(-1), minlength=R3)
    del warm
    lo.set_hot_rows(hot_rows_by_frequency(counts, C))
    idx = zipf_selections(B, K, R3, seed=5, perm=perm, device=dev).to(torch.int32)
    gq = torch.Generator().manual_seed(0)
    q = torch.randn(B, H, D, generator=gq).to(torch.bfloat16).to(dev)
    hit = lo.hit_rate(idx)
    out = torch.empty(B, H, 512, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(B, H, dtype=torch.float32, device=dev)
    _settle(lambda: lo.attend(q, idx, SM_SCALE, 1.0, H, out=out, lse=lse))
    ms = _timed(lambda: lo.attend(q, idx, SM_SCALE, 1.0, H, out=out, lse=lse), steps, max(2, a.warmup // 4))
    o_t, l_t = lo.attend(q, idx, SM_SCALE, 1.0, H, return_lse=True)
    # single-tier check: the same rows gathered into HBM and attended in one pass
    staged = torch.empty(B * K, ROWB, dtype=torch.uint8, device=dev)
    if compact:
        kernels.row400_gather(lo.host, idx.reshape(-1).to(torch.int64), staged)
    else:
        kernels.gather(lo.host, idx.reshape(-1).to(torch.int64), staged)
    sidx = torch.arange(B * K, dtype=torch.int32, device=dev).view(B, K)
    o_1, l_1 = kernels.attend(q, staged, sidx, SM_SCALE)
    torch.cuda.synchronize()
    d_o = float((o_t.float() - o_1.float()).abs().max())
    d_l = float((l_t - l_1).abs().max())
    # host-tier roofline: pinned host -> HBM copy bandwidth
    hb = torch.empty(1 << 28, dtype=torch.uint8, pin_memory=True)
    db = torch.empty(1 << 28, dtype=torch.uint8, device=dev)
    h2d_ms = _timed(lambda: db.copy_(hb, non_blocking=True), 5, 2)
    h2d = (1 << 28) / (h2d_ms * 1e-3) / 1e9
    miss_bytes = (1.0 - hit) * B * K * HOST_ROW[row_fmt]
    gbs = ALG_BYTES / (ms * 1e-3) / 1e9
    res = {"value": round(gbs, 3), "unit": "GB/s (algorithmic bytes of the config-2 step / step time)",
           "ms_per_step": round(ms, 4), "hit_rate": round(hit, 4), "host_rows_per_step": int(round((1 - hit) * B * K)),
           "pcie_bytes_per_step": int(miss_bytes), "pcie_gbs_achieved": round(miss_bytes / (ms * 1e-3) / 1e9, 2),
           "h2d_copy_gbs": round(h2d, 2), "max_abs_diff_vs_single_tier": {"out": d_o, "lse": d_l},
           "host_row_format": row_fmt, "cache_line_format": cache_fmt, "host_rows_read_in_place": host_direct,
           "workload": "BASELINE config 3: B=64, H=128, top-2048 Zipf(1.1) rows of a 2,097,152-row "
                       + ("compact Row400 (e2m2b32)" if compact else "Row656") +
                       " pool in pinned host memory, HBM hot set = 524,288 most frequent rows over 64 warm-up steps "
                       + ("(compact Row400 lines in HBM, decoded into Row656 staging each step)" if cache_fmt == "e2m2"
                          else "(Row656 in HBM)") + "; tier split -> HBM-tier attention + host rows gathered over PCIe"
                       + (" and decoded" if compact else "") + " -> host-tier attention -> LSE merge"
                       + (" (host_direct: no staging copy, the host-tier attention reads the pinned rows over PCIe)"
                          if host_direct else "")}
    del lo, hb, db, staged
    torch.cuda.empty_cache()
    return res


def run_config3_ways(a, dev, steps=None, row_fmt="e2m2", W=16, two=False, cache_fmt="row656", C=None):
    """Config 3 shapes with the dynamic W-way cache in place of the static hot set: every step draws fresh Zipf(1.1)
    selections (a decode stream); the cache is warmed over the 64 warm-up steps' draws, then each timed step looks
    its rows up, places the misses, copies them in over PCIe (beside the attention over the hits) and attends.
    two: two-choice set placement (a miss whose set is full takes a way in a second, hashed set); cache_fmt "e2m2":
    compact Row400 lines (the reference's production mode with row_fmt "e2m2", W = 8 and two); C: cache lines
    (default a quarter of the pool)."""
    import torch
    from arcagi2_flashnext_dots3_amd.sparse_offload import HOST_ROW, LayerOffload
    steps = steps or a.steps
    warm_n = max(2, a.warmup // 4)
    C = int(C or R3 // 4)
    lo = LayerOffload(R3, dev, cache_rows=C, row_fmt=row_fmt, cache_mode="ways", ways=W, spill_rows=B * K,
                      two_choice=two, cache_fmt=cache_fmt)
    _cache_fill(lo.host, R3, 1, dev, fmt=2 if row_fmt == "e2m2" else 0)
    perm = torch.randperm(R3, generator=torch.Generator().manual_seed(3))
    gq = torch.Generator().manual_seed(0)
    q = torch.randn(B, H, D, generator=gq).to(torch.bfloat16).to(dev)
    out = torch.empty(B, H, 512, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(B, H, dtype=torch.float32, device=dev)
    warm = zipf_selections(64 * B, K, R3, seed=4, perm=perm, device=dev).to(torch.int32).view(64, B, K)
    for s_ in range(64):
        lo.attend(q, warm[s_], SM_SCALE, 1.0, H, out=out, lse=lse)
    del warm
    # stats pass over fresh steps (untimed): hits, misses, spills per step from the cache's counters
    nstat = 8
    stat = zipf_selections(nstat * B, K, R3, seed=6, perm=perm, device=dev).to(torch.int32).view(nstat, B, K)
    hits = misses = spills = 0
    for s_ in range(nstat):
        lo.attend(q, stat[s_], SM_SCALE, 1.0, H, out=out, lse=lse)
        st = lo.wc.state.cpu()
        hits += int(st[3]); misses += int(st[1]); spills += int(st[2])
    del stat
    nsteps = warm_n + steps
    seq = zipf_selections(nsteps * B, K, R3, seed=5, perm=perm, device=dev).to(torch.int32).view(nsteps, B, K)
    it = iter(range(nsteps))
    ms = _timed(lambda: lo.attend(q, seq[next(it)], SM_SCALE, 1.0, H, out=out, lse=lse), steps, warm_n)
    hb = torch.empty(1 << 28, dtype=torch.uint8, pin_memory=True)      # host-tier roofline: pinned -> HBM copy
    db = torch.empty(1 << 28, dtype=torch.uint8, device=dev)
    h2d = (1 << 28) / (_timed(lambda: db.copy_(hb, non_blocking=True), 5, 2) * 1e-3) / 1e9
    del hb, db
    hit = hits / (nstat * B * K)
    mb = misses / nstat * HOST_ROW[row_fmt]
    res = {"value": round(ALG_BYTES / (ms * 1e-3) / 1e9, 3),
           "unit": "GB/s (algorithmic bytes of the config-2 step / step time)", "ms_per_step": round(ms, 4),
           "hit_rate": round(hit, 4), "misses_per_step": round(misses / nstat, 1),
           "spill_rows_per_step": round(spills / nstat, 1), "pcie_bytes_per_step": int(mb),
           "pcie_gbs_achieved": round(mb / (ms * 1e-3) / 1e9, 2), "h2d_copy_gbs": round(h2d, 2),
           "host_row_format": row_fmt, "cache_line_format": cache_fmt, "ways": W, "two_choice": bool(two),
           "cache_lines": C,
           "workload": f"config 3 shapes with a dynamic {W}-way set-associative{' two-choice' * two} HBM cache of "
                       f"{C:,} {'compact Row400' if cache_fmt == 'e2m2' else 'Row656'} lines (+ 131,072 spill rows) "
                       f"over a 2,097,152-row "
                       f"{'compact Row400' if row_fmt == 'e2m2' else 'Row656'}"
                       " pinned host pool; each step a fresh Zipf(1.1) draw of B=64 x top-2048 rows; warmed over "
                       "64 steps; per step: lookup / place / resolve, miss copy over PCIe beside the attention over "
                       "the hits, attention over the fresh rows merged in its epilogue"}
    del lo, seq
    torch.cuda.empty_cache()
    return res


# ------------------------------------------------------------------------------------------------ config 4
def run_config4(a, dev):
    import numpy as np
    import torch
    from arcagi2_flashnext_dots3_amd import kernels
    from arcagi2_flashnext_dots3_amd.shard_indexer import ShardStore
    bs = 64
    results = {}
    for L in (32768, 131072):
        nbp = L // bs
        kc = torch.empty(B * nbp, bs, 132, dtype=torch.uint8, device=dev)
        st = ShardStore(kc, 1, 0)
        g = torch.Generator(device=dev).manual_seed(5)
        chunk = 1 << 20
        for r0 in range(0, B * L, chunk):
            n = min(chunk, B * L - r0)
            k = torch.randn(n, 128, generator=g, device=dev).to(torch.bfloat16)
            st.write(k, torch.arange(r0, r0 + n, dtype=torch.int64, device=dev), False)
        bt = torch.arange(B * nbp, dtype=torch.int32, device=dev).view(B, nbp)
        q = torch.randn(B, 64, 128, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16).to(dev)
        w = torch.rand(B, 64, generator=torch.Generator().manual_seed(7)).to(dev)
        req = torch.arange(B, dtype=torch.int32, device=dev)
        ctx = torch.full((B,), L, dtype=torch.int32, device=dev)
        lg = torch.empty(B, L, dtype=torch.float32, device=dev)
        lg16 = torch.empty(B, L, dtype=torch.float16, device=dev)
        out = torch.empty(B, K, dtype=torch.int32, device=dev)

        def logits(dst=lg):
            kernels._lib.call("spmla_index_logits", q.data_ptr(), q.stride(0), q.stride(1), w.data_ptr(),
                              w.stride(0), kc.data_ptr(), st.R_local, st.RPB, st.STRIDE_BLK, bt.data_ptr(),
                              bt.stride(0), bs, req.data_ptr(), ctx.data_ptr(), B, 64, 128, L, 1, 0, 1,
                              dst.data_ptr(), dst.stride(0), int(dst.dtype == torch.float16), kernels._stream(q))

        # eager (host dispatch from Python included) and from HIP graphs of 20 launches (the launches alone;
        # the top-k is four kernels per call)
        ms_l = _graph_ms(logits, a.steps, a.warmup, reps=20)
        ms_t = _graph_ms(lambda: kernels.topk(lg, ctx, K, out=out), a.steps, a.warmup, reps=20)
        ms_l_eager = _timed(logits, a.steps, a.warmup)      # after the graph timings, at their settled clocks
        ms_t_eager = _timed(lambda: kernels.topk(lg, ctx, K, out=out), a.steps, a.warmup)
        # the reference's fp16 logits mode (ARC_SHARD_F16OUT): fp16 logits, top-k on fp16 keys
        ms_l16 = _graph_ms(lambda: logits(lg16), a.steps, a.warmup, reps=20)
        ms_t16 = _graph_ms(lambda: kernels.topk(lg16, ctx, K, out=out), a.steps, a.warmup, reps=20)
        # the step as ShardStore.logits_topk runs it at P = 1: the top-k's first histogram built in the logits
        # epilogue (spmla_index_logits_hist), then the top-k without its histogram pass (spmla_topk_ws_prehist)
        ws = torch.empty(int(kernels._lib.lib().spmla_topk_ws_bytes(B, L, K)), dtype=torch.uint8, device=dev)

        def fused(dst=lg):
            if kernels.logits_hist(q, w, kc, st.R_local, st.RPB, st.STRIDE_BLK, bt, bs, req, ctx, L, K, dst, ws,
                                   noinf=True):
                kernels.topk_prehist(dst, ctx, K, ws, out=out)
            else:                        # a top-k chunk of 65536 or more columns: the separate calls
                logits(dst)
                kernels.topk(dst, ctx, K, out=out, ws=ws)

        fused()
        torch.cuda.synchronize()
        out_f = out.clone()
        kernels.topk(lg, ctx, K, out=out)
        torch.cuda.synchronize()
        fused_same = bool(torch.equal(out_f, out))
        ms_f = _graph_ms(fused, a.steps, a.warmup, reps=20)
        ms_f16 = _graph_ms(lambda: fused(lg16), a.steps, a.warmup, reps=20)
        key_bytes = B * L * 132
        alg = key_bytes + B * 64 * 128 * 2 + B * 64 * 4 + B * L * 4
        flops = B * L * 64 * 128 * 2
        cpu = None
        if not a.no_cpu and L == 32768:
            cpu = _cpu_indexer(q, w, kc, B, L, bt, bs)
        results[str(L)] = {"step_us": round(ms_f * 1e3, 2), "separate_step_us": round((ms_l + ms_t) * 1e3, 2),
                           "fused_matches_separate": fused_same, "logits_us": round(ms_l * 1e3, 2),
                           "topk_us": round(ms_t * 1e3, 2), "logits_eager_us": round(ms_l_eager * 1e3, 2),
                           "topk_eager_us": round(ms_t_eager * 1e3, 2),
                           "logits_gbs": round(alg / (ms_l * 1e-3) / 1e9, 1),
                           "logits_hbm_frac": round(alg / (ms_l * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                           "logits_tflops": round(flops / (ms_l * 1e-3) / 1e12, 1),
                           "topk_read_gbs": round(B * L * 4 / (ms_t * 1e-3) / 1e9, 1),
                           "alg_bytes": alg, "cpu_baseline": cpu,
                           "f16_logits": {"step_us": round(ms_f16 * 1e3, 2),
                                          "separate_step_us": round((ms_l16 + ms_t16) * 1e3, 2),
                                          "logits_us": round(ms_l16 * 1e3, 2), "topk_us": round(ms_t16 * 1e3, 2),
                                          "note": "the reference's ARC_SHARD_F16OUT mode: selection on fp16 logits"}}
        del kc, lg, lg16, ws
        torch.cuda.empty_cache()
    r = results["32768"]
    roof = {"bound": "hbm", "achieved": r["logits_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": r["logits_hbm_frac"], "traffic": None, "kernel": "spmla::idx::logits_kernel"}
    return _line("indexer logits + top-2048 step us, B=64, 64 heads x 128, L=32768", r["step_us"], "us", a,
                 r["step_us"] / 1e3, "e4m3 keys x bf16 q: bf16 MFMA, fp32 accumulate",
                 {"workload": "BASELINE config 4: indexer top-2048 of L = 32768 and 131072, B=64"}, roof,
                 r["cpu_baseline"], hib=False, by_ctx=results)


def _cpu_indexer(q, w, kc, Bn, L, bt, bs):
    """torch-CPU restatement (fp32) of the indexer step: dequantized keys, sum_h w relu(q k) * s, topk; one
    sequence timed (median of 3), scaled to B sequences."""
    import torch
    from oracle import cpu_port
    nt = cpu_port.threads()
    torch.set_num_threads(nt)
    rows = kc.view(-1, 132)[bt[0].long().repeat_interleave(bs) * bs + torch.arange(L, device=kc.device) % bs].cpu()
    tab = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float()
    kk = tab[rows[:, :128].long()] * rows[:, 128:132].contiguous().view(torch.float32)
    qh, wh = q[0].float().cpu(), w[0].cpu()
    ts = []
    for _ in range(3):
        t0 = time.perf_counter()
        s = (torch.relu(qh @ kk.T) * wh[:, None]).sum(0)
        torch.topk(s, K)
        ts.append(time.perf_counter() - t0)
    t = sorted(ts)[1] * Bn
    return {"value": round(t * 1e6, 1), "unit": "us per step (B=64 scaled from one sequence)", "cores": nt,
            "kind": "port", "sample": f"one sequence of L={L} keys in fp32 torch, median of 3, x{Bn}"}


# ------------------------------------------------------------------------------------------------ config 5
def run_config5(a, dev):
    import torch
    from arcagi2_flashnext_dots3_amd import kernels
    NQ, CTXMAX, bs = 8192, 65536, 64
    nblk = CTXMAX // bs + 64
    cache = torch.zeros(nblk, bs, ROWB, dtype=torch.uint8, device=dev)
    gb = torch.Generator().manual_seed(10)
    bt = torch.randperm(nblk, generator=gb)[: CTXMAX // bs].to(torch.int32).view(1, -1).to(dev)
    pos0 = CTXMAX - NQ
    posp = torch.arange(pos0, device=dev)
    prior = (bt[0, posp // bs].long() * bs + posp % bs)
    g = torch.Generator(device=dev).manual_seed(1)
    for r0 in range(0, pos0, 1 << 16):
        n = min(1 << 16, pos0 - r0)
        kernels.cache_write(torch.randn(n, 512, generator=g, device=dev).to(torch.bfloat16),
                            torch.randn(n, 64, generator=g, device=dev).to(torch.bfloat16), prior[r0:r0 + n], cache)
    g9 = torch.Generator(device=dev).manual_seed(9)
    kv = torch.randn(NQ, 512, generator=g9, device=dev).to(torch.bfloat16)
    pe = torch.randn(NQ, 64, generator=g9, device=dev).to(torch.bfloat16)
    posn = torch.arange(pos0, CTXMAX, device=dev)
    slots = bt[0, posn // bs].long() * bs + posn % bs
    _settle(lambda: kernels.cache_write(kv, pe, slots, cache))
    ms_w = _timed(lambda: kernels.cache_write(kv, pe, slots, cache), a.steps, a.warmup)
    g8 = torch.Generator().manual_seed(8)
    tk = torch.stack([torch.randperm(min(p + 1, CTXMAX), generator=g8)[:K] for p in range(pos0, CTXMAX)])
    tk = tk.to(torch.int32).to(dev)
    rows = kernels.rows_from_topk(tk, torch.zeros(NQ, dtype=torch.int32, device=dev), bt, bs)
    q = torch.randn(NQ, H, D, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16).to(dev)
    out = torch.empty(NQ, H, 512, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(NQ, H, dtype=torch.float32, device=dev)
    flat = cache.view(-1, ROWB)
    _settle(lambda: kernels.attend(q, flat, rows, SM_SCALE, out=out, lse=lse))
    ms_a = _timed(lambda: kernels.attend(q, flat, rows, SM_SCALE, out=out, lse=lse), max(3, a.steps // 20),
                  max(1, a.warmup // 10))
    flops = NQ * H * K * (2 * 576 + 2 * 512)
    tf = flops / (ms_a * 1e-3) / 1e12
    wb = NQ * (1024 + 128 + 8) + NQ * ROWB
    # the offload prefill's staging gather (dsa_sm89.py:341-345): the chunk's distinct selected rows copied from the
    # HBM cache into a dense staging area (one 656-byte read and write per row)
    uniq = torch.unique(rows[rows >= 0].long())
    staged = torch.empty(uniq.numel(), ROWB, dtype=torch.uint8, device=dev)
    ms_g = _timed(lambda: kernels.gather(flat, uniq, staged), a.steps, a.warmup)
    gb = 2 * uniq.numel() * ROWB
    cpu = None
    if not a.no_cpu:
        from oracle import cpu_port
        nt = cpu_port.threads()
        torch.set_num_threads(nt)
        ns = 256
        rh = flat[rows[:ns].clamp(min=0).reshape(-1).long()].cpu()
        li = torch.arange(ns * K, dtype=torch.int32).view(ns, K)
        qh = q[:ns].cpu()
        t0 = time.perf_counter()
        cpu_port.attention_f32(qh, rh, li, SM_SCALE)
        t = (time.perf_counter() - t0) * NQ / ns
        cpu = {"value": round(t * 1e3, 1), "unit": "ms per prefill chunk (attention only)", "cores": nt,
               "kind": "port", "sample": f"{ns} of {NQ} queries in fp32 torch, scaled linearly"}
    roof = {"bound": "mfma", "achieved": round(tf, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tf / BF16_PEAK_TFLOPS, 4), "traffic": None, "kernel": "spmla::attn::fwd_kernel"}
    res = _line("chunked prefill attention ms (8192 queries x 128 heads x top-2048) + cache write us", ms_a, "ms", a,
                ms_a + ms_w, "f16 MFMA (QK latent and PV), bf16 MFMA (rope), fp32 accumulate",
                {"workload": "BASELINE config 5: 8192 queries, 128 heads, top-2048 of <= 65536 prior rows; write "
                             "8192 rows at random slots of a paged cache (block 64)"}, roof, cpu, hib=False,
                cache_write_us=round(ms_w * 1e3, 2),
                cache_write_gbs=round(wb / (ms_w * 1e-3) / 1e9, 1),
                staging_gather_rows=int(uniq.numel()), staging_gather_us=round(ms_g * 1e3, 2),
                staging_gather_gbs=round(gb / (ms_g * 1e-3) / 1e9, 1))
    return res


# ------------------------------------------------------------------------------------------------ config 1
def _graphed(fn, reps):
    """`reps` calls of fn captured into one HIP graph (torch.cuda.CUDAGraph; the library's entry points launch on
    torch's current stream, which is the capture stream inside torch.cuda.graph). Returns the graph's replay. One
    graph launch costs about as much as a few-microsecond kernel, so a decode loop's graph holds many launches."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    torch.cuda.synchronize()
    return g.replay


def _graph_ms(fn, steps, warmup, reps=50):
    """Average ms of one fn() call replayed from graphs of `reps` calls (at least `steps` calls timed)."""
    replay = _graphed(fn, reps)
    n = max(1, (steps + reps - 1) // reps)
    _settle(replay)
    return _timed(replay, n, max(1, warmup // reps)) / reps


def run_config6(a, dev):
    """The steps either side of the decode attention at config-2 shapes (B = 64 tokens, H = 128 heads): the fused
    query build q[t, h] = (q_nope @ W_UK_T[h], q_pe) and the output matmul attn_out @ W_UV[h], both on FP8
    block-scaled weights (128 x 512 per head and direction). Beside it: torch.bmm on the bf16 weights they replace.
    A decode loop replays its launches from a HIP graph; each side is timed that way (the host-side dispatch of a
    few-microsecond launch from Python would otherwise be what is measured) and eagerly for reference."""
    import torch
    from arcagi2_flashnext_dots3_amd import kernels
    N, T, P, L, V = H, B, 128, 512, 128
    g = torch.Generator().manual_seed(9)
    cu = (torch.randn(N, L, P, generator=g) * 60).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).to(dev)
    su = (torch.exp(torch.randn(N, P, L // 128, generator=g)) * 1e-3).to(dev)
    cv = (torch.randn(N, V, L, generator=g) * 60).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).to(dev)
    sv = (torch.exp(torch.randn(N, V, L // 128, generator=g)) * 1e-3).to(dev)
    q_nope = torch.randn(T, N, P, generator=g).to(torch.bfloat16).to(dev)
    q_pe = torch.randn(T, N, 64, generator=g).to(torch.bfloat16).to(dev)
    x = torch.randn(T, N, L, generator=g).to(torch.bfloat16).to(dev)
    q = torch.empty(T, N, D, dtype=torch.bfloat16, device=dev)
    y = torch.empty(T, N, V, dtype=torch.bfloat16, device=dev)

    def query():
        kernels.mla_query(q_nope, q_pe, cu, su, out=q)

    def output():
        kernels.bmm_fp8(x.transpose(0, 1), cv, sv, True, y.transpose(0, 1))

    def step():
        query()
        output()

    step()
    torch.cuda.synchronize()
    q_e, y_e = q.clone(), y.clone()
    eager_ms = _timed(step, a.steps, a.warmup)
    replay = _graphed(step, 1)
    q.zero_()
    y.zero_()
    for _ in range(3):                                  # every replay reproduces the eager result
        replay()
        torch.cuda.synchronize()
        if not (torch.equal(q, q_e) and torch.equal(y, y_e)):
            raise SystemExit("config 6: graph replay differs from the eager step")
    ms = _graph_ms(step, a.steps, a.warmup)
    q_us = _graph_ms(query, a.steps, a.warmup) * 1e3
    v_us = _graph_ms(output, a.steps, a.warmup) * 1e3
    # bytes: FP8 codes + fp32 block scales + activations in and out
    qb = N * L * P + su.numel() * 4 + T * N * P * 2 + T * N * 64 * 2 + T * N * D * 2
    vb = N * V * L + sv.numel() * 4 + T * N * L * 2 + T * N * V * 2
    flops = 2 * T * N * L * P * 2
    # the bf16 path they replace: torch.bmm on dequantized bf16 weights (twice the weight bytes), also graphed
    wu = (cu.view(torch.float8_e4m3fn).float() * su.repeat_interleave(128, 2).transpose(1, 2)).to(torch.bfloat16)
    wv = (cv.view(torch.float8_e4m3fn).float() * sv.repeat_interleave(128, 2)).to(torch.bfloat16)
    wu_t = wu.transpose(1, 2).contiguous()                  # [N, P, L]
    wv_t = wv.transpose(1, 2).contiguous()                  # [N, L, V]
    qn_h = q_nope.transpose(0, 1).contiguous()
    x_h = x.transpose(0, 1).contiguous()

    def step_bf16():
        torch.cat([torch.bmm(qn_h, wu_t).transpose(0, 1), q_pe], dim=2)
        torch.bmm(x_h, wv_t)

    ms_bf16 = _graph_ms(step_bf16, a.steps, a.warmup)
    ms_bf16_eager = _timed(step_bf16, a.steps, a.warmup)
    gbs = (qb + vb) / (ms * 1e-3) / 1e9
    return _line("MLA absorbed matmuls (query build + output), FP8 weights, B=64 H=128, us per decode step", ms * 1e3,
                 "us", a, ms, "e4m3 weights dequantized to bf16, bf16 MFMA, fp32 accumulate",
                 {"workload": "q[t,h] = (q_nope @ W_UK_T[h], q_pe) into the [64, 128, 576] attention query + "
                              "attn_out @ W_UV[h] -> [64, 128, 128]; per head 128 x 512 FP8 weights each way, "
                              "128 x 128 block scales; steps replayed from HIP graphs of 50"},
                 {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                  "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                  "kernel": "spmla::mla::bmm_fp8_staged_kernel"},
                 hib=False, query_build_us=round(q_us, 2), output_bmm_us=round(v_us, 2),
                 eager_us=round(eager_ms * 1e3, 2), alg_bytes=qb + vb,
                 tflops=round(flops / (ms * 1e-3) / 1e12, 2), torch_bf16_bmm_us=round(ms_bf16 * 1e3, 2),
                 torch_bf16_bmm_eager_us=round(ms_bf16_eager * 1e3, 2))


def run_config7(a, dev):
    """MTP decode at the config-2 shapes: B = 16 requests x 4 MTP tokens (64 tokens), 128 heads, top-2048 each of a
    32768-row context per request; the tokens of a request share ~95% of their rows (union ~2450 of 4 x 2048, the
    reference's observed ~2400). The request-packed path (the union of each request's rows, then one attention
    over the union per request and head group) against the per-token attention over the same selections; both
    timed from HIP graphs, the packed one including its union kernel."""
    import torch
    from arcagi2_flashnext_dots3_amd import kernels
    NRQ, QL = 16, 4
    T = NRQ * QL
    R = NRQ * CTX
    pool = torch.empty(R, ROWB, dtype=torch.uint8, device=dev)
    _cache_fill(pool, R, 1, dev)
    g = torch.Generator(device=dev).manual_seed(11)
    base = torch.stack([torch.randperm(CTX, generator=g, device=dev)[:K] for _ in range(NRQ)]) + \
        torch.arange(NRQ, device=dev)[:, None] * CTX                            # [NRQ, K]
    idx = base.repeat_interleave(QL, 0).clone()                               # [T, K]
    own = torch.stack([torch.randperm(CTX, generator=g, device=dev)[:K] for _ in range(T)]) + \
        (torch.arange(T, device=dev) // QL)[:, None] * CTX
    swap = torch.rand(T, K, generator=g, device=dev) < 0.05
    idx = torch.where(swap, own, idx)
    srt = torch.sort(idx, dim=1).values                                     # duplicates within a token -> -1
    dup = torch.zeros_like(srt, dtype=torch.bool)
    dup[:, 1:] = srt[:, 1:] == srt[:, :-1]
    idx = torch.where(dup, torch.full_like(srt, -1), srt).to(torch.int32).contiguous()
    q = torch.randn(T, H, D, generator=torch.Generator().manual_seed(12)).to(torch.bfloat16).to(dev)
    out = torch.empty(T, H, 512, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(T, H, dtype=torch.float32, device=dev)
    u, mk, cnt = kernels.mtp_union(idx, ql=QL, R=R)

    def packed():
        un = kernels.mtp_union(idx, ql=QL, R=R)
        kernels.attend_packed(q, pool, idx, SM_SCALE, ql=QL, out=out, lse=lse, union=un)

    def per_token():
        kernels.attend(q, pool, idx, SM_SCALE, out=out, lse=lse)

    packed()
    torch.cuda.synchronize()
    o_p, l_p = out.clone(), lse.clone()
    per_token()
    torch.cuda.synchronize()
    diff = float(((out.float() - o_p.float()).abs() / out.float().abs().clamp_min(1.0)).max())
    ms = _graph_ms(packed, a.steps, a.warmup, reps=20)
    ms_tok = _graph_ms(per_token, a.steps, a.warmup, reps=20)
    ms_union = _graph_ms(lambda: kernels.mtp_union(idx, ql=QL, R=R), a.steps, a.warmup, reps=20)
    rows_loaded = int(cnt.sum())
    return _line("MTP request-packed sparse-MLA decode step us, 16 requests x 4 tokens, ctx32K top2048", ms * 1e3, "us",
                 a, ms, "fp8e4m3 rows x bf16 q: bf16 MFMA (QK), f16 MFMA (PV), fp32 accumulate",
                 {"workload": "16 requests x 4 MTP tokens, 128 heads, top-2048 per token of a 32768-row context, ~95% "
                              "of a request's rows shared; union then packed attention (graph of 20 steps)"},
                 {"bound": "hbm", "achieved": round(rows_loaded * ROWB / (ms * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBS,
                  "unit": "GB/s", "frac": round(rows_loaded * ROWB / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                  "traffic": None, "kernel": "spmla::pk::attn_kernel<true>"},
                 hib=False, per_token_us=round(ms_tok * 1e3, 2), union_us=round(ms_union * 1e3, 2),
                 union_rows_per_request=round(rows_loaded / NRQ, 1), rows_per_request_per_token=K * QL,
                 max_rel_diff_vs_per_token=round(diff, 5))


def run_config1(a, dev):
    import numpy as np
    import torch
    from arcagi2_flashnext_dots3_amd import kernels
    from oracle import cpu_port
    T1, H1, R1, K1 = 1, 16, 4096, 256
    pool = torch.empty(R1, ROWB, dtype=torch.uint8, device=dev)
    _cache_fill(pool, R1, 1, dev)
    q = torch.randn(T1, H1, D, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16).to(dev)
    idx = torch.randperm(R1, generator=torch.Generator().manual_seed(2))[:K1].to(torch.int32).view(1, K1).to(dev)
    ms = _timed(lambda: kernels.attend(q, pool, idx, SM_SCALE), a.steps, a.warmup)
    o, l = kernels.attend(q, pool, idx, SM_SCALE)
    ph, qh, ih = pool.cpu(), q.cpu(), idx.cpu()
    eo, el = cpu_port.attention_f32(qh, ph, ih, SM_SCALE)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(20):
        cpu_port.attention_f32(qh, ph, ih, SM_SCALE)
    tc = (time.perf_counter() - t0) / 20
    alg = K1 * ROWB + H1 * D * 2 + H1 * 512 * 2 + H1 * 4 + K1 * 4
    return _line("sparse-MLA decode us, B=1, 16 heads, top-256 of 4096", ms * 1e3, "us", a, ms,
                 "bf16 MFMA, fp32 accumulate", {"workload": "BASELINE config 1"},
                 {"bound": "hbm", "achieved": round(alg / (ms * 1e-3) / 1e9, 2), "peak": HBM_PEAK_GBS,
                  "unit": "GB/s", "frac": round(alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 5), "traffic": None},
                 {"value": round(tc * 1e6, 1), "unit": "us", "cores": cpu_port.threads(), "kind": "port",
                  "sample": "the full config-1 step, mean of 20"}, hib=False,
                 max_abs_diff_vs_fp32_cpu={"out": float((o.float().cpu() - eo).abs().max()),
                                           "lse": float((l.cpu() - el).abs().max())})


def _child_variant(args, timeout=600):
    """Run this script with `args` in a child process (a plain subprocess) and return the `detail` of the JSON line it
    prints, or an error record; the primary line must still print."""
    import subprocess
    try:
        r = subprocess.run([sys.executable, os.path.abspath(__file__)] + args, capture_output=True, text=True,
                           timeout=timeout)
        lines = [ln for ln in r.stdout.splitlines() if ln.startswith("{")]
        if r.returncode != 0 or not lines:
            return {"error": f"exit {r.returncode}: {(r.stderr or r.stdout)[-300:]}"}
        return json.loads(lines[-1]).get("detail", {})
    except Exception as e:
        return {"error": repr(e)[:300]}


# the reference's shipped offload mode as config-3 options (mode_submit.json: ARC_OFFLOAD_WAYS=8, ROW_FMT=e2m2, CCACHE=1,
# OVERLAP=1, TWO_CHOICE=1)
PRODUCTION = ["--host-rows", "e2m2", "--cache", "ways", "--ways", "8", "--two-choice", "--cache-fmt", "e2m2"]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-variant", action="store_true", help="config 2 only: skip the host-tier (config 3) variant")
    ap.add_argument("--config", type=int, default=2, choices=[1, 2, 3, 4, 5, 6, 7])
    ap.add_argument("--host-rows", default="row656", choices=["row656", "e2m2"],
                    help="config 3: host pool row format (Row656, or the reference's compact Row400 e2m2b32 rows)")
    ap.add_argument("--cache", default="static", choices=["static", "ways"],
                    help="config 3: static frequency hot set (BASELINE's definition) or the dynamic W-way cache")
    ap.add_argument("--ways", type=int, default=16, help="config 3 --cache ways: lines per set")
    ap.add_argument("--two-choice", action="store_true", help="config 3 --cache ways: two-choice set placement")
    ap.add_argument("--cache-rows", type=int, default=0,
                    help="config 3 --cache ways: cache lines (default a quarter of the pool, 524,288)")
    ap.add_argument("--cache-fmt", default="row656", choices=["row656", "e2m2"],
                    help="config 3 with --host-rows e2m2: Row656 cache lines, or compact Row400 lines in HBM")
    ap.add_argument("--host-direct", action="store_true",
                    help="config 3 static cache, Row656 host rows: the host-tier attention reads the pinned rows in "
                         "place over PCIe instead of a staging copy into HBM")
    ap.add_argument("--copy-calib", type=int, default=0, metavar="BYTES",
                    help="only run 5 plain device-to-device copies of BYTES bytes (the reference kernel for scaling "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE readings) and exit")
    ap.add_argument("--no-traffic", action="store_true",
                    help="config 2: skip the in-run rocprofv3 FETCH_SIZE / WRITE_SIZE counting of roofline.traffic")
    ap.add_argument("--probe", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--rows", type=int, default=656, choices=[656, 576],
                    help="config 2: 576 times the step over a Row576 cache alone (the row576_variant of the default line)")
    ap.add_argument("--idx-sets", type=int, default=4,
                    help="steps rotate over this many independent top-k draws; 4 sets select 344 MB of rows, more "
                         "than the 256 MB Infinity Cache, so rows come from HBM rather than from the previous step")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU only (one GPU's share of the path); --gpus {a.gpus} is not "
              f"supported", file=sys.stderr)
        sys.exit(2)
    import torch
    dev = torch.device("cuda:0")
    if a.copy_calib:
        src = torch.ones(a.copy_calib, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calib_bytes": a.copy_calib}), flush=True)
        return
    if a.config == 2 and a.rows == 576:         # config 2 over the plugin's Row576 cache alone (profiling)
        gq = torch.Generator().manual_seed(0)
        q = torch.randn(B, H, D, generator=gq).to(torch.bfloat16).to(dev)
        idxs = []
        for n in range(a.idx_sets):
            gi = torch.Generator().manual_seed(2 + n)
            idxs.append(torch.stack([torch.randperm(CTX, generator=gi)[:K] + b * CTX for b in range(B)])
                        .to(torch.int32).to(dev))
        out = torch.empty(B, H, 512, dtype=torch.bfloat16, device=dev)
        lse = torch.empty(B, H, dtype=torch.float32, device=dev)
        r = run_row576(a, dev, q, idxs, out, lse)
        res = _line(METRIC, r["gbs"], "GB/s", a, r["step_us"] / 1e3, "fp8e4m3 rows x bf16 q: bf16 MFMA (QK), f16 MFMA (PV)",
                    {"workload": r["workload"]}, {"bound": "hbm", "achieved": r["gbs"], "peak": HBM_PEAK_GBS,
                                                  "unit": "GB/s", "frac": r["frac"], "traffic": None,
                                                  "kernel": r["kernel"]}, detail=r)
    elif a.config == 2 and a.probe:
        print(json.dumps(run_probe(a, dev)), flush=True)
        return
    elif a.config == 2:
        res = run_config2(a, dev)
        if not a.no_variant:
            # each config-3 variant in a fresh child process (its own GPU context and pinned pool), so no variant
            # inherits the allocator and pinned-memory state of the ones before it
            st = str(min(a.steps, 20))
            for key, extra in (("host_tier_variant", ["--host-rows", "row656"]),
                               ("host_tier_compact_variant", ["--host-rows", "e2m2"]),
                               ("host_tier_compact_cache_variant", ["--host-rows", "e2m2", "--cache-fmt", "e2m2"]),
                               ("host_tier_production_variant", PRODUCTION),
                               ("host_tier_overflow_one_choice_variant",
                                [x for x in PRODUCTION if x != "--two-choice"] + ["--cache-rows", "131072"]),
                               ("host_tier_overflow_two_choice_variant", PRODUCTION + ["--cache-rows", "131072"])):
                print(f"[bench] {key}: child process", file=sys.stderr, flush=True)
                res[key] = _child_variant(["--config", "3", "--steps", st, "--warmup", str(a.warmup)] + extra)
    elif a.config == 3:
        r = run_config3_ways(a, dev, row_fmt=a.host_rows, W=a.ways, two=a.two_choice, cache_fmt=a.cache_fmt,
                             C=a.cache_rows) if a.cache == "ways" else \
            run_config3(a, dev, row_fmt=a.host_rows, cache_fmt=a.cache_fmt, host_direct=a.host_direct)
        res = _line("offload split-K decode step us (host tier + HBM hot rows), B=64 top2048", r["ms_per_step"] * 1e3,
                    "us", a, r["ms_per_step"], "bf16 MFMA, fp32 accumulate", {"workload": r["workload"]},
                    {"bound": "pcie", "achieved": r["pcie_gbs_achieved"], "peak": r["h2d_copy_gbs"], "unit": "GB/s",
                     "frac": round(r["pcie_gbs_achieved"] / max(r["h2d_copy_gbs"], 1e-9), 4), "traffic": None},
                    hib=False, detail=r)
    elif a.config == 4:
        res = run_config4(a, dev)
    elif a.config == 5:
        res = run_config5(a, dev)
    elif a.config == 7:
        res = run_config7(a, dev)
    elif a.config == 6:
        res = run_config6(a, dev)
    else:
        res = run_config1(a, dev)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
