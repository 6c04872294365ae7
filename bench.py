"""Benchmark of the MI355X sparse-MLA decode step (BASELINE.json metric: "sparse-MLA decode step us + effective GB/s
(% of 8 TB/s), B=64 ctx32K top2048").

Default workload = BASELINE config 2 (all-HBM decode): B = 64 sequences, 128 query heads, 32768-token context per
sequence held as Row656 KV rows in HBM (latent / rope N(0,1), written by the library's own cache-write kernel),
q bf16 N(0,1), top-2048 row indices per sequence drawn uniformly without replacement, softmax scale 1/sqrt(192),
bf16 out + fp32 LSE. One step = one spmla_attn_splitk launch over the whole batch (inputs resident in HBM).

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

Prints ONE JSON line. `value` = effective GB/s = algorithmic bytes of the step / measured step time, where the
algorithmic bytes are 131072 rows x 656 B + q + idx + out + lse = 104,366,080 B. `roofline` is measured live with
HIP events on the stream the kernel is launched on; `cpu_baseline` times the float32 torch-CPU restatement
(oracle/cpu_port.py) of the same full step on this host's cores.
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


def build_inputs(dev, nsets=1):
    import torch
    from arcagi2_flashnext_dots3_amd import kernels
    R = B * CTX
    pool = torch.empty(R, ROWB, dtype=torch.uint8, device=dev)
    g = torch.Generator(device=dev).manual_seed(1)
    chunk = 1 << 18
    for r0 in range(0, R, chunk):
        n = min(chunk, R - r0)
        kv = torch.randn(n, 512, generator=g, device=dev).to(torch.bfloat16)
        pe = torch.randn(n, 64, generator=g, device=dev).to(torch.bfloat16)
        slots = torch.arange(r0, r0 + n, dtype=torch.int64, device=dev)
        kernels.cache_write(kv, pe, slots, pool)
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
    return {"value": ALG_BYTES / t / 1e9, "unit": "GB/s", "cores": nt, "kind": "port",
            "sample": f"full config-2 step (B=64, H=128, K=2048) in fp32 torch on {nt} threads, median of 5: "
                      f"{t * 1e3:.1f} ms/step"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--idx-sets", type=int, default=4,
                    help="steps rotate over this many independent top-k draws; 4 sets select 344 MB of rows, more "
                         "than the 256 MB Infinity Cache, so rows come from HBM rather than from the previous step")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU only (one GPU's share of the path); --gpus {a.gpus} is not "
              f"supported", file=sys.stderr)
        sys.exit(2)
    import torch
    from arcagi2_flashnext_dots3_amd import kernels
    dev = torch.device("cuda:0")
    pool, q, idxs = build_inputs(dev, a.idx_sets)
    out = torch.empty(B, H, 512, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(B, H, dtype=torch.float32, device=dev)

    cur = [0]

    def step():
        kernels.attend(q, pool, idxs[cur[0] % len(idxs)], SM_SCALE, out=out, lse=lse)
        cur[0] += 1

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream(dev)            # the stream spmla_attn_splitk is launched on
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(a.steps):
        step()
    e1.record(st)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / a.steps
    gbs = ALG_BYTES / (ms * 1e-3) / 1e9
    res = {
        "metric": "sparse-MLA decode step us + effective GB/s (% of 8 TB/s), B=64 ctx32K top2048",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms, 5), "step_us": round(ms * 1e3, 2), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp8e4m3 x bf16 MFMA, fp32 accumulate", "data": "synthetic (seeded N(0,1))",
        "config": {"workload": "BASELINE config 2: all-HBM sparse-MLA decode, B=64, H=128, ctx=32768/seq, "
                               "top-2048, Row656 rows, bf16 out + fp32 LSE",
                   "global_batch": B, "heads": H, "ctx": CTX, "topk": K, "row_bytes": ROWB,
                   "idx_sets": a.idx_sets, "attn_teams": int(os.environ.get("SPMLA_ATTN_TEAMS", "2"))},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "spmla::attn::attn_kernel", "alg_bytes_per_launch": ALG_BYTES,
                     "mfma_tflops": round(ALG_FLOPS / (ms * 1e-3) / 1e12, 2),
                     "mfma_frac_bf16_peak": round(ALG_FLOPS / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4)},
        "cpu_baseline": None,
    }
    tf = os.environ.get("SPMLA_TRAFFIC_JSON")   # optional: HBM bytes per launch measured by rocprofv3 --pmc
    if tf and os.path.exists(tf):
        res["roofline"]["traffic"] = json.load(open(tf)).get("attn_kernel_bytes")
    if not a.no_cpu:
        res["cpu_baseline"] = cpu_baseline(pool, q, idxs[0])
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
