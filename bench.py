"""Benchmark of the batched sampler on one MI355X.

Workload: BASELINE.json config 2 (the north star) -- 64 rows x 151,936 f32
logits N(0, 3^2) with 5 ids/row boosted by +8, per-row history counts from
1,024 Zipf(1.1) ids, presence 1.5 + repetition 1.05, T 0.7, top-k 20,
top-p 0.8, one uniform per row.  A step is one fg_sampler_hip_sample launch
over one batch.  Inputs are generated on the device with torch (synthetic) and
rotated over >= 4 GB of distinct batches so the 256 MB Infinity Cache cannot
hold them: every step reads its logits and counts from HBM.

Output: one JSON line (see the repository's bench contract), with
`roofline` (dominant kernel: algorithmic bytes / HIP-event launch time vs the
8 TB/s HBM peak) and `cpu_baseline` (the C oracle on the host cores over a
bounded sample of the same batch).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "flash-gordon_amd"))

VOCAB = 151_936
ROWS = 64
HBM_PEAK_GBS = 8000.0
ALG_BYTES_PER_ROW = 8 * VOCAB  # f32 logit + u32 count, each read once
METRIC = "sampled rows/sec @ vocab 151,936, batch 64; achieved HBM GB/s vs peak"
TRAFFIC_FILE = ROOT / "profiles" / "sample_rows_config2_traffic.json"


def make_sets(torch, dev, nsets, seed=1002):
    """Device-side synthetic batches of config 2."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    ranks = torch.arange(1, VOCAB + 1, device=dev, dtype=torch.float64)
    zipf = ranks.pow(-1.1)
    zipf = (zipf / zipf.sum()).float()
    logits, counts, uniforms = [], [], []
    for _ in range(nsets):
        x = torch.randn((ROWS, VOCAB), generator=g, device=dev) * 3.0
        boost = torch.randint(0, VOCAB, (ROWS, 5), generator=g, device=dev)
        x.scatter_add_(1, boost, torch.full((ROWS, 5), 8.0, device=dev))
        perm = torch.randperm(VOCAB, generator=g, device=dev)
        hist = perm[torch.multinomial(zipf.expand(ROWS, VOCAB), 1024, replacement=True, generator=g)]
        c = torch.zeros((ROWS, VOCAB), dtype=torch.int32, device=dev)
        c.scatter_add_(1, hist, torch.ones_like(hist, dtype=torch.int32))
        u = torch.rand(ROWS, generator=g, device=dev)
        logits.append(x.contiguous())
        counts.append(c.contiguous())
        uniforms.append(u)
    return logits, counts, uniforms


def configs(fg_hip):
    return [fg_hip.make_config(0.7, 0.8, 20, presence=1.5, repetition=1.05)] * ROWS


def cpu_baseline(x, c, u, gpu_tokens, budget_s):
    """The C oracle (oracle/, a restatement of the reference semantics) on this
    host's cores over a bounded sample of batch 0; also cross-checks the GPU's
    tokens for that batch."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import numpy as np
    import oracle_ffi as O

    cfg = [dict(temperature=0.7, top_p=0.8, top_k=20, presence=1.5, frequency=0.0,
                repetition=1.05)] * ROWS
    ref = O.sample_rows(cfg, x, u, counts=c, threads=1)
    same = (ref["token"] == gpu_tokens) | (ref["margin"] < 1e-6)
    parity = f"{int(same.sum())}/{ROWS} rows match the oracle (bit-exact ids, 1e-6 boundary clause)"

    def timed(threads, budget):
        rows = 0
        t0 = time.perf_counter()
        while True:
            O.sample_rows(cfg, x, u, counts=c, threads=threads)
            rows += ROWS
            el = time.perf_counter() - t0
            if el >= budget:
                return rows / el, rows, el

    single, rows1, el1 = timed(1, budget_s / 2)
    threads = min(16, len(os.sched_getaffinity(0)))
    multi, rows_n, el_n = timed(threads, budget_s / 2)
    return {
        "value": round(multi, 1), "unit": "rows/s", "cores": threads, "kind": "port",
        "sample": (f"batch 0 of the bench workload (64 rows x 151,936), repeated: {rows_n} rows "
                   f"in {el_n:.1f} s on {threads} threads; single core {single:.1f} rows/s "
                   f"({rows1} rows in {el1:.1f} s)"),
        "single_core_value": round(single, 1),
    }, parity


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--set-gb", type=float, default=4.0, help="distinct input bytes to rotate over")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only a 1 GiB device copy (the rocprof FETCH/WRITE_SIZE reference)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only; the rows of a batch are independent "
              "and would shard data-parallel over GPUs with no exchange (see DESIGN.md).",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import fg_hip

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.calibrate_copy:
        # A plain copy kernel of known size: 1 GiB read + 1 GiB written per
        # launch; its counters scale the sampler's FETCH_SIZE / WRITE_SIZE.
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "copy", "bytes_read": src.numel() * 4,
                          "bytes_written": dst.numel() * 4, "launches": args.steps}))
        return
    set_bytes = ROWS * ALG_BYTES_PER_ROW
    nsets = max(4, int(args.set_gb * 1e9 / set_bytes + 0.999))
    logits, counts, uniforms = make_sets(torch, dev, nsets)
    torch.cuda.synchronize()

    sampler = fg_hip.HipSampler(VOCAB, ROWS)
    stream = torch.cuda.current_stream()
    sampler.set_configs(configs(fg_hip), stream=stream.cuda_stream)
    tokens = torch.empty((nsets, ROWS), dtype=torch.int32, device=dev)
    status = torch.empty((nsets, ROWS), dtype=torch.int32, device=dev)

    def step(i):
        k = i % nsets
        sampler.sample(logits[k], uniforms[k], tokens[k], counts=counts[k], row_status=status[k],
                       stream=stream.cuda_stream)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for i in range(args.steps):
        step(i)
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(end)
    per_launch_s = ms / 1e3 / args.steps
    rows_per_s = ROWS * args.steps / (ms / 1e3)
    achieved = set_bytes / per_launch_s / 1e9
    assert int((status != 0).sum()) == 0, "rows reported errors"

    traffic = None
    if TRAFFIC_FILE.exists():
        traffic = json.loads(TRAFFIC_FILE.read_text()).get("hbm_bytes_per_launch")

    line = {
        "metric": METRIC,
        "value": round(rows_per_s, 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (device-generated config-2 batches, rotated over "
                f"{nsets} distinct sets = {nsets * set_bytes / 1e9:.2f} GB)",
        "config": {"workload": "config 2: 64 rows x 151,936 f32 logits, presence 1.5 + repetition "
                               "1.05 over 1,024 Zipf(1.1) history ids, T 0.7, top-k 20, top-p 0.8",
                   "rows": ROWS, "vocab": VOCAB, "global_batch": ROWS, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "kernel": "fg::sample_rows_kernel<true>",
                     "algorithmic_bytes_per_launch": set_bytes,
                     "launch_us": round(per_launch_s * 1e6, 3)},
        "wall_s": round(wall, 3),
    }
    if not args.no_cpu:
        g_tok = tokens[0].cpu().numpy().view("uint32")
        cpu, parity = cpu_baseline(logits[0].cpu().numpy(), counts[0].cpu().numpy().view("uint32"),
                                   uniforms[0].cpu().numpy(), g_tok, args.cpu_seconds)
        line["cpu_baseline"] = cpu
        line["parity"] = parity
    print(json.dumps(line))


if __name__ == "__main__":
    main()
