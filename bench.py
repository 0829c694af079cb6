"""Benchmark of the batched sampler on one MI355X.

Default workload: BASELINE.json config 2 (the north star) -- 64 rows x
151,936 f32 logits N(0, 3^2) with 5 ids/row boosted by +8, per-row history
counts from 1,024 Zipf(1.1) ids, presence 1.5 + repetition 1.05, T 0.7,
top-k 20, top-p 0.8, one uniform per row.  A step is one fg_sampler_hip_sample
call over one batch (one kernel launch; two for whole-row nucleus batches).
Inputs are generated on the device with torch (synthetic, same shapes and
distributions as the configs) and rotated over >= 4 GB of distinct batches so
the 256 MB Infinity Cache cannot hold them: every step reads its logits and
counts from HBM.

`--split WAYS` (2 or 4) times instead what the output owner's GPU does per
token in the reference's vocabulary-split greedy output: its slice of each
row reduced to one finalist (fg_hip_output_slice_reduce) and the finalists
of all ways combined (fg_hip_output_split_combine); the other ways'
finalists are reduced once, untimed, as the other ranks would send them.

`--lm-head` times the producer of the logits instead: the reference's LM
head (248,320 x 2,560 Q8_0 weights in the cooked layout, random bytes with
binary16 scales in [1e-3, 2e-2]) times `--tokens` hidden vectors, fused with
each token's greedy finalist (fg_hip_output_slice_run_dense, ways 1).

`--config N` times the other configurations of BASELINE.json the same way
(1: one greedy row; 3: 256 rows, whole-row nucleus; 4: 128 rows, quantised
logits, greedy or sampled; 5: 1,024 rows with top-20 log-probs).  The driver
runs the default.

Output: one JSON line (see the repository's bench contract), with `roofline`
(dominant kernel: algorithmic bytes / HIP-event launch time vs the 8 TB/s HBM
peak), `parity` (batch 0 checked against the C oracle; the run fails on a
mismatch) and `cpu_baseline` (the C oracle on every host core over a bounded
sample of the same batch, with the single-core figure beside it).
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


class cfg(dict):
    """One row's controls as the oracle's dict; `.c` is the C struct the
    sampler takes."""

    def __init__(self, fg_hip, t, p, k, pres=0.0, freq=0.0, rep=1.0):
        super().__init__(temperature=t, top_p=p, top_k=k, presence=pres, frequency=freq,
                         repetition=rep)
        self.c = fg_hip.make_config(t, p, k, presence=pres, frequency=freq, repetition=rep)


def zipf_counts(torch, g, dev, rows, draws, perm, vocab=VOCAB):
    """Per-row u32 counts of `draws` Zipf(1.1) token ids (rank -> id by a
    permutation), as the configs' history tables."""
    ranks = torch.arange(1, vocab + 1, device=dev, dtype=torch.float64)
    zipf = ranks.pow(-1.1)
    zipf = (zipf / zipf.sum()).float()
    hist = perm[torch.multinomial(zipf.expand(rows, vocab), draws, replacement=True, generator=g)]
    c = torch.zeros((rows, vocab), dtype=torch.int32, device=dev)
    c.scatter_add_(1, hist, torch.ones_like(hist, dtype=torch.int32))
    return c


class Workload:
    """One BASELINE.json configuration: row count, per-row controls, input
    generator and the algorithmic bytes of one step."""

    def __init__(self, cid, fg_hip, sampled=True):
        self.cid = cid
        self.flags = 0
        self.logprobs = 0
        self.penalised_rows = None
        if cid == 1:
            self.rows = 1
            self.configs = [cfg(fg_hip, 0.0, 1.0, 1, rep=1.05)]
            self.name = "config 1: 1 row x 151,936, repetition 1.05 over 64 history ids, greedy"
        elif cid == 2:
            self.rows = ROWS
            self.configs = [cfg(fg_hip, 0.7, 0.8, 20, pres=1.5, rep=1.05)] * ROWS
            self.name = ("config 2: 64 rows x 151,936 f32 logits, presence 1.5 + repetition "
                         "1.05 over 1,024 Zipf(1.1) history ids, T 0.7, top-k 20, top-p 0.8")
        elif cid == 3:
            self.rows = 256
            self.configs = [cfg(fg_hip, 1.0, 0.95, 0, pres=0.5, freq=0.3)] * 256
            self.flags = fg_hip.ALLOW_FULL_VOCAB
            self.name = ("config 3: 256 rows x 151,936, 2*Student-t(3), presence 0.5 + frequency "
                         "0.3 over 8,192 Zipf history ids, T 1.0, top-p 0.95 over the whole row")
        elif cid == 4:
            self.rows = 128
            self.penalised_rows = 64
            mk = ((lambda rep: cfg(fg_hip, 0.8, 0.9, 50, rep=rep)) if sampled
                  else (lambda rep: cfg(fg_hip, 0.0, 1.0, 1, rep=rep)))
            self.configs = [mk(1.1)] * 64 + [mk(1.0)] * 64
            self.name = ("config 4: 128 rows x 151,936 quantised logits, rows 0-63 repetition 1.1 "
                         "over 256 history ids, " + ("top-k 50, top-p 0.9" if sampled else "greedy"))
        elif cid == 5:
            self.rows = 1024
            self.configs = [cfg(fg_hip, 0.6, 0.95, 64, pres=1.0, freq=0.2, rep=1.05)] * 1024
            self.logprobs = 20
            self.name = ("config 5: 1,024 rows x 151,936, N(0,2^2)/N(0,6^2), presence 1.0 + "
                         "frequency 0.2 + repetition 1.05 over 32,768 Zipf history ids, T 0.6, "
                         "top-k 64, top-p 0.95, top-20 log-probs")
        else:
            raise SystemExit(f"bench.py: unknown --config {cid}")
        # Algorithmic bytes: 4 B logit for every element, 4 B count for rows
        # with penalties, plus the per-row outputs of config 5.
        pen = self.rows if self.penalised_rows is None else self.penalised_rows
        self.alg_bytes = 4 * VOCAB * self.rows + 4 * VOCAB * pen
        if cid == 5:
            self.alg_bytes += self.rows * (4 + 4 + 20 * 8)

    def make(self, torch, dev, g):
        """One device batch: (logits, counts, uniforms)."""
        rows = self.rows
        perm = torch.randperm(VOCAB, generator=g, device=dev)
        if self.cid in (1, 2):
            x = torch.randn((rows, VOCAB), generator=g, device=dev) * 3.0
            if self.cid == 2:
                boost = torch.randint(0, VOCAB, (rows, 5), generator=g, device=dev)
                x.scatter_add_(1, boost, torch.full((rows, 5), 8.0, device=dev))
                c = zipf_counts(torch, g, dev, rows, 1024, perm)
            else:
                ids = torch.randint(0, VOCAB, (rows, 64), generator=g, device=dev)
                c = torch.zeros((rows, VOCAB), dtype=torch.int32, device=dev)
                c.scatter_add_(1, ids, torch.ones_like(ids, dtype=torch.int32))
        elif self.cid == 3:
            z = torch.randn((rows, VOCAB), generator=g, device=dev)
            chi = torch.distributions.Chi2(torch.tensor(3.0, device=dev)).sample((rows, VOCAB))
            x = 2.0 * z / torch.sqrt(chi / 3.0)
            c = zipf_counts(torch, g, dev, rows, 8192, perm)
        elif self.cid == 4:
            x = (torch.randn((rows, VOCAB), generator=g, device=dev) * 3.0 / 0.25).round() * 0.25
            x = x.clamp(-16.0, 16.0)
            spike = torch.randint(0, VOCAB, (rows, 1), generator=g, device=dev)
            x.scatter_(1, spike, torch.full((rows, 1), 20.0, device=dev))
            ids = torch.randint(0, VOCAB, (rows, 256), generator=g, device=dev)
            c = torch.zeros((rows, VOCAB), dtype=torch.int32, device=dev)
            c.scatter_add_(1, ids, torch.ones_like(ids, dtype=torch.int32))
        else:
            sig = torch.where(torch.arange(rows, device=dev) % 2 == 0, 2.0, 6.0).unsqueeze(1)
            x = torch.randn((rows, VOCAB), generator=g, device=dev) * sig
            c = zipf_counts(torch, g, dev, rows, 32768, perm)
        u = torch.rand(rows, generator=g, device=dev)
        return x.float().contiguous(), c.contiguous(), u


def host_cores():
    return len(os.sched_getaffinity(0))


def oracle_parity(w, x, c, u, gpu_tokens, gpu_status, lp=None):
    """Batch 0 of the run checked against the C oracle (oracle/, a restatement
    of the reference semantics): token ids bit-exact unless the oracle's draw
    lies within 1e-6 of a cumulative-probability boundary, row status equal,
    log-probs within 1e-5.  Raises on any mismatch."""
    import numpy as np
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle_ffi as O

    ref = O.sample_rows(list(w.configs), x, u, counts=c, logprobs=w.logprobs,
                        threads=host_cores())
    assert (ref["status"] == gpu_status).all(), "row status differs from the oracle"
    same = (ref["token"] == gpu_tokens) | (ref["margin"] < 1e-6)
    assert same.all(), f"{int((~same).sum())}/{w.rows} rows differ from the oracle"
    if lp is not None:
        vals, ids = lp
        err = float(np.abs(vals - ref["lp_values"]).max())
        assert err <= 1e-5, f"log-probs differ from the oracle by {err}"
        # Ids may swap only between equal values.
        swapped = ids != ref["lp_ids"]
        assert (np.abs(vals - ref["lp_values"])[swapped] <= 1e-5).all()
    return (f"{w.rows}/{w.rows} rows of batch 0 match the oracle "
            f"(bit-exact ids, 1e-6 boundary clause: {int((ref['token'] != gpu_tokens).sum())} used)")


def cpu_baseline(w, x, c, u, budget_s):
    """The C oracle timed on this host's cores over a bounded sample of
    batch 0: half the budget on every core the process may run on, half on
    one core."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle_ffi as O

    cfgs = list(w.configs)

    def timed(threads, budget):
        rows = 0
        t0 = time.perf_counter()
        while True:
            O.sample_rows(cfgs, x, u, counts=c, logprobs=w.logprobs, threads=threads)
            rows += w.rows
            el = time.perf_counter() - t0
            if el >= budget:
                return rows / el, rows, el

    single, rows1, el1 = timed(1, budget_s / 2)
    threads = host_cores()
    multi, rows_n, el_n = timed(threads, budget_s / 2)
    return {
        "value": round(multi, 1), "unit": "rows/s", "cores": threads, "kind": "port",
        "sample": (f"batch 0 of the bench workload ({w.rows} rows x 151,936), repeated: "
                   f"{rows_n} rows in {el_n:.1f} s on all {threads} host cores; single core "
                   f"{single:.1f} rows/s ({rows1} rows in {el1:.1f} s)"),
        "single_core_value": round(single, 1),
    }


LM_VOCAB, LM_WIDTH = 248_320, 2_560


def lm_head_bench(args, torch, fg_hip, dev):
    tokens = args.tokens
    tile = fg_hip.lib().fg_q8_0_cooked_tile_bytes(LM_WIDTH)
    nbytes = fg_hip.lib().fg_q8_0_cooked_matrix_bytes(LM_WIDTH, LM_VOCAB)
    tiles = nbytes // tile
    g = torch.Generator(device=dev)
    g.manual_seed(38)
    w = torch.randint(0, 256, (tiles, tile), dtype=torch.uint8, device=dev, generator=g)
    scales = 16 * (LM_WIDTH // 32)
    d = (torch.rand((tiles, scales), device=dev, generator=g) * 0.019 + 0.001).to(torch.float16)
    w[:, :2 * scales] = d.view(torch.uint8)
    x = torch.randn((tokens, LM_WIDTH), device=dev, generator=g)
    sl = fg_hip.OutputSlice(LM_VOCAB, 1, 0, LM_VOCAB, max(tokens, 1))
    vals = torch.empty(tokens, device=dev)
    ids = torch.empty(tokens, dtype=torch.int32, device=dev)
    status = torch.empty(tokens, dtype=torch.int32, device=dev)
    logits = torch.empty(tokens * LM_VOCAB, device=dev)
    stream = torch.cuda.current_stream()
    if args.sampled:
        # Config 2's controls and history statistics at the LM head's vocabulary.
        ctl = [fg_hip.make_config(0.7, 0.8, 20, presence=1.5, repetition=1.05)] * tokens
        perm = torch.randperm(LM_VOCAB, generator=g, device=dev)
        counts = zipf_counts(torch, g, dev, tokens, 1024, perm, vocab=LM_VOCAB)
        uniforms = torch.rand(tokens, generator=g, device=dev)

    def step():
        if args.unfused:
            fg_hip.dense_q8_0_cooked(logits, w, x, LM_WIDTH, LM_VOCAB, tokens,
                                     stream=stream.cuda_stream)
        elif args.sampled:
            sl.run_dense_sampled(w, x, LM_WIDTH, tokens, ctl, uniforms, ids, vals, status,
                                 counts=counts, stream=stream.cuda_stream)
        else:
            sl.run_dense(w, x, LM_WIDTH, tokens, vals, ids, status, stream=stream.cuda_stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(args.steps):
        step()
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(end)
    per_s = ms / 1e3 / args.steps
    if args.sampled:
        # The same tokens from the unfused path: plain product, then the sampler.
        fg_hip.dense_q8_0_cooked(logits, w, x, LM_WIDTH, LM_VOCAB, tokens, stream=stream.cuda_stream)
        smp = fg_hip.HipSampler(LM_VOCAB, tokens)
        smp.set_configs(ctl, stream=stream.cuda_stream)
        want = torch.empty(tokens, dtype=torch.int32, device=dev)
        smp.sample(logits.view(tokens, LM_VOCAB), uniforms, want, counts=counts,
                   stream=stream.cuda_stream)
        torch.cuda.synchronize()
        assert bool((ids == want).all()), "fused sampled tokens differ from the unfused path"
        assert int(status.abs().sum()) == 0
    elif not args.unfused:
        fg_hip.dense_q8_0_cooked(logits, w, x, LM_WIDTH, LM_VOCAB, tokens, stream=stream.cuda_stream)
        y = logits.view(tokens, LM_VOCAB)
        torch.cuda.synchronize()
        assert bool((ids.to(torch.int64) == torch.argmax(y, dim=1)).all()), "finalist != argmax"
        assert int(status.abs().sum()) == 0
    # Algorithmic bytes: the weights and inputs once, the logits written when
    # unfused, the history counts read when sampled.
    alg = (nbytes + 4 * LM_WIDTH * tokens + (4 * LM_VOCAB * tokens if args.unfused else 0)
           + (4 * LM_VOCAB * tokens if args.sampled else 0))
    kernel = ("fg::dense_q8_cooked_kernel" if args.unfused else
              "fg::dense_q8_sample_kernel" if args.sampled else "fg::dense_q8_finalist_kernel")
    what = ("logits" if args.unfused else
            "fused penalties + top-k 20 + top-p 0.8 + draw" if args.sampled else
            "fused greedy finalist")
    print(json.dumps({
        "metric": f"LM-head tokens/sec (Q8_0 {LM_VOCAB} x {LM_WIDTH}, {what})",
        "value": round(tokens / per_s, 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms / args.steps, 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "q8_0 x f32",
        "data": "synthetic (random Q8_0 bytes, binary16 scales in [1e-3, 2e-2], N(0,1) hidden)",
        "config": {"workload": f"lm-head-{'plain' if args.unfused else 'sampled' if args.sampled else 'finalist'}-t{tokens}",
                   "rows": LM_VOCAB, "width": LM_WIDTH, "tokens": tokens,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(alg / per_s / 1e9, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(alg / per_s / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": None, "kernel": kernel, "algorithmic_bytes_per_launch": alg,
                     "launch_us": round(per_s * 1e6, 3)},
        "wall_s": round(wall, 3)}))


def timed(args, torch, stream, step):
    """W untimed, then K timed calls of step() on `stream` (HIP events)."""
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(args.steps):
        step()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3 / args.steps, time.perf_counter() - t0


def history_bench(args, torch, fg_hip, dev):
    """Count tables of config 2's batch rebuilt from FG_MSG_OUTPUT_HISTORY
    payloads on the device (64 rows x 151,936, 1,024 Zipf(1.1) history ids
    per row), the output-history path's per-session reset for a whole batch.
    Algorithmic bytes: the cleared tables (4 B per count) plus the payloads."""
    import numpy as np
    rows, hist = ROWS, 1024
    rng = np.random.default_rng(38)
    ranks = np.arange(1, VOCAB + 1, dtype=np.float64)
    p = ranks ** -1.1
    p /= p.sum()
    perm = rng.permutation(VOCAB)
    payloads = [fg_hip.history_encode(perm[rng.choice(VOCAB, hist, p=p)], session_slot=0, vocab=VOCAB)
                for _ in range(rows)]
    offsets = np.zeros(rows + 1, dtype=np.int64)  # u64 byte offsets (the C signature)
    offsets[1:] = np.cumsum([len(x) for x in payloads])
    blob = torch.from_numpy(np.frombuffer(b"".join(payloads), dtype=np.uint8).copy()).to(dev)
    d_off = torch.from_numpy(offsets).to(dev)
    counts = torch.empty((rows, VOCAB), dtype=torch.int32, device=dev)
    status = torch.empty(rows, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream()
    per_s, wall = timed(args, torch, stream, lambda: fg_hip.history_build_wire(
        counts, VOCAB, VOCAB, blob, d_off, rows, status, stream=stream.cuda_stream))
    assert int(status.abs().sum()) == 0
    assert int(counts.sum()) == rows * hist
    alg = 4 * rows * VOCAB + int(offsets[-1]) + 8 * (rows + 1)
    print(json.dumps({
        "metric": "history tables rebuilt/sec (64 rows x 151,936 from wire payloads)",
        "value": round(1 / per_s, 1), "unit": "batches/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(per_s * 1e3, 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u32",
        "data": "synthetic (1,024 Zipf(1.1) ids per row, seeded permutation of ranks)",
        "config": {"workload": "history-build-wire-config2", "rows": rows, "vocab": VOCAB,
                   "history": hist, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(alg / per_s / 1e9, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(alg / per_s / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": None, "kernel": "fg::history_wire_build_kernel",
                     "algorithmic_bytes_per_launch": alg, "launch_us": round(per_s * 1e6, 3)},
        "wall_s": round(wall, 3)}))


def topk_reduce_bench(args, torch, fg_hip, dev):
    """The QSA top-512 scan (src/qsa.c:839-851) over 262,144 scores in one
    fg_hip_topk_reduce_all launch; the per-level ladder it replaces (one
    fg_hip_topk_reduce per level, 262,144 -> 32,768 -> 4,096 -> 512) is timed
    beside it and must give the same 512 entries.  Algorithmic bytes per
    launch: the scores read once and the 512 outputs (score, id) written."""
    count = 262_144
    g = torch.Generator(device=dev)
    g.manual_seed(39)
    scores = torch.randn(count, device=dev, generator=g)
    bufs = [(torch.empty(count // 8, device=dev), torch.empty(count // 8, dtype=torch.int32, device=dev))
            for _ in range(2)]
    work = torch.zeros(fg_hip.topk_reduce_all_workspace_bytes(count), dtype=torch.uint8, device=dev)
    out_s = torch.empty(512, device=dev)
    out_i = torch.empty(512, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream()

    def ladder():
        s, ids, n, slot = scores, None, count, 0
        while n > 512:
            ls, li = bufs[slot]
            n = fg_hip.topk_reduce(ls, li, s, ids, n, stream=stream.cuda_stream)
            s, ids, slot = ls, li, slot ^ 1
        return s, ids

    def step():
        fg_hip.topk_reduce_all(out_s, out_i, scores, None, count, work, stream=stream.cuda_stream)

    ladder_s, _ = timed(args, torch, stream, ladder)
    per_s, wall = timed(args, torch, stream, step)
    ls, li = ladder()
    step()
    torch.cuda.synchronize()
    want = torch.topk(scores, 512).values
    assert torch.equal(out_s, want), "top-512 differs from torch.topk"
    assert torch.equal(out_i, li[:512]) and torch.equal(out_s, ls[:512]), "differs from the ladder"
    alg = count * 4 + 512 * 8
    print(json.dumps({
        "metric": "QSA top-512 scans/sec (262,144 scores)",
        "value": round(1 / per_s, 1), "unit": "scans/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(per_s * 1e3, 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (N(0,1) scores, ids implicit)",
        "config": {"workload": "qsa-top512-one-launch", "count": count, "parallelism": "single GPU"},
        "ladder_us": round(ladder_s * 1e6, 3),
        "roofline": {"bound": "hbm", "achieved": round(alg / per_s / 1e9, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(alg / per_s / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": None, "kernel": "fg::topk_reduce_all_kernel",
                     "algorithmic_bytes_per_launch": alg, "launch_us": round(per_s * 1e6, 3)},
        "wall_s": round(wall, 3)}))


def split_bench(args, torch, fg_hip, dev, w, sets, nsets, batch_bytes):
    ways, rows = args.split, w.rows
    quarter = VOCAB // ways
    spans = [(i * quarter, quarter if i + 1 < ways else VOCAB - i * quarter) for i in range(ways)]
    slices = [fg_hip.OutputSlice(VOCAB, ways, f, n, rows) for f, n in spans]
    stream = torch.cuda.current_stream()
    sid = stream.cuda_stream
    parts_v = torch.empty((nsets, ways, rows), dtype=torch.float32, device=dev)
    parts_i = torch.empty((nsets, ways, rows), dtype=torch.int32, device=dev)
    parts_s = torch.empty((nsets, ways, rows), dtype=torch.int32, device=dev)
    for k in range(nsets):  # the other ranks' finalists, reduced once
        for way in range(1, ways):
            f, n = spans[way]
            slices[way].reduce(sets[k][0][:, f:f + n], parts_v[k, way], parts_i[k, way],
                               parts_s[k, way], stride=VOCAB, stream=sid)
    ranks = torch.tensor([0] + [(4, 0, 1, 2)[i] for i in range(1, ways)], dtype=torch.uint8,
                         device=dev).repeat(rows)
    pv = torch.empty((nsets, rows, ways), dtype=torch.float32, device=dev)
    pi = torch.empty((nsets, rows, ways), dtype=torch.int32, device=dev)
    tokens = torch.empty((nsets, rows), dtype=torch.int32, device=dev)
    status = torch.zeros((nsets, rows), dtype=torch.int32, device=dev)
    own = spans[0][1]

    def step(i, sid):  # the owner's step: its slice reduced and combined, one launch
        k = i % nsets
        slices[0].reduce_combine(sets[k][0][:, :own], pv[k], pi[k], ranks, spans, tokens[k],
                                 None, status[k], stride=VOCAB, stream=sid)

    # The gathered [row][way] finalists are filled once from the untimed
    # reductions plus the owner's own reduction of the same set.
    for k in range(nsets):
        slices[0].reduce(sets[k][0][:, :own], parts_v[k, 0], parts_i[k, 0], parts_s[k, 0],
                         stride=VOCAB, stream=sid)
    pv.copy_(parts_v.transpose(1, 2))
    pi.copy_(parts_i.transpose(1, 2))
    # Launches of a few us are shorter than their host-side call, so the
    # timed steps are replays of a captured HIP graph of `per_graph` steps
    # (the kernels use no memset; the one-launch step's epochs live on the
    # device, so replays stay exact).
    per_graph = 100
    steps = max(per_graph, args.steps // per_graph * per_graph)
    for i in range(args.warmup):
        step(i, sid)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cap = torch.cuda.current_stream().cuda_stream
        for i in range(per_graph):
            step(i, cap)
    graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps // per_graph):
        graph.replay()
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(end)
    per_step_s = ms / 1e3 / steps
    x = sets[0][0]
    want = torch.argmax(x, dim=1)  # finite N(0, 9) rows: the argmax is unique a.s.
    assert bool((tokens[0] == want.to(torch.int32)).all()) and int(status.sum()) == 0
    alg = 4 * own * rows
    print(json.dumps({
        "metric": f"split-output owner steps/sec ({ways}-way, vocab {VOCAB}, batch {rows})",
        "value": round(1.0 / per_step_s, 1), "unit": "steps/s", "n_gpus": 1,
        "steps": steps, "warmup": args.warmup, "ms_per_step": round(ms / steps, 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": f"synthetic (config-{args.config} logits, {nsets} rotated sets)",
        "config": {"workload": f"split{ways}-owner-{w.name}", "rows": rows, "vocab": VOCAB,
                   "slice_rows": own, "parallelism": "single GPU (one rank's share)",
                   "launches_per_step": 1},
        "roofline": {"bound": "hbm", "achieved": round(alg / per_step_s / 1e9, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(alg / per_step_s / 1e9 / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "fg::slice_owner_kernel (grids resident at once) or "
                               "fg::slice_row_kernel (the library picks)",
                     "algorithmic_bytes_per_launch": alg,
                     "launch_us": round(per_step_s * 1e6, 3)},
        "wall_s": round(wall, 3)}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--config", type=int, default=2, help="BASELINE.json configuration (1-5)")
    ap.add_argument("--greedy", action="store_true", help="config 4: the greedy run")
    ap.add_argument("--set-gb", type=float, default=4.0, help="distinct input bytes to rotate over")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--split", type=int, default=0, choices=(0, 2, 4),
                    help="time the owner's side of the vocabulary-split greedy output")
    ap.add_argument("--lm-head", action="store_true",
                    help="time the Q8_0 LM-head product fused with the greedy finalist")
    ap.add_argument("--tokens", type=int, default=1, help="--lm-head: hidden vectors per step")
    ap.add_argument("--unfused", action="store_true",
                    help="--lm-head: the plain product writing logits (no finalist)")
    ap.add_argument("--sampled", action="store_true",
                    help="--lm-head: fused with config 2's penalties, top-k, top-p and draw")
    ap.add_argument("--per-step-configs", action="store_true",
                    help="upload every row's controls before every sample (the owner loop)")
    ap.add_argument("--history", action="store_true",
                    help="time the history count tables rebuilt from wire payloads")
    ap.add_argument("--topk-reduce", action="store_true",
                    help="time the QSA top-512 scan over 262,144 scores (one launch, ladder beside it)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only a 1 GiB device copy (the rocprof FETCH/WRITE_SIZE reference)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only; the rows of a batch are independent "
              "and would shard data-parallel over GPUs with no exchange.",
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

    if args.lm_head:
        return lm_head_bench(args, torch, fg_hip, dev)
    if args.history:
        return history_bench(args, torch, fg_hip, dev)
    if args.topk_reduce:
        return topk_reduce_bench(args, torch, fg_hip, dev)

    w = Workload(args.config, fg_hip, sampled=not args.greedy)
    batch_bytes = 8 * VOCAB * w.rows
    nsets = max(2, int(args.set_gb * 1e9 / batch_bytes + 0.999))
    g = torch.Generator(device=dev)
    g.manual_seed(1000 + args.config)
    sets = [w.make(torch, dev, g) for _ in range(nsets)]
    torch.cuda.synchronize()

    if args.split:
        return split_bench(args, torch, fg_hip, dev, w, sets, nsets, batch_bytes)

    sampler = fg_hip.HipSampler(VOCAB, w.rows)
    stream = torch.cuda.current_stream()
    sampler.set_configs([c.c for c in w.configs], flags=w.flags, stream=stream.cuda_stream)
    # Sentinels: a set the run never reaches keeps them, and only the sets
    # the run wrote are checked.
    tokens = torch.full((nsets, w.rows), -1, dtype=torch.int32, device=dev)
    status = torch.full((nsets, w.rows), -12345, dtype=torch.int32, device=dev)
    L = w.logprobs
    lpv = torch.empty((nsets if L else 1, w.rows, max(L, 1)), dtype=torch.float32, device=dev)
    lpi = torch.empty((nsets if L else 1, w.rows, max(L, 1)), dtype=torch.int32, device=dev)

    # --per-step-configs: the output owner's loop, where every row's controls
    # arrive with every token (src/protocol.c:1158-1166): fresh controls are
    # uploaded before each sample, alternating between the workload's and a
    # second set of the same kind (other temperatures and top-p values).
    ctl_sets = [[c.c for c in w.configs],
                [fg_hip.make_config(c["temperature"] * 0.9 if c["temperature"] else 0.0,
                                    min(1.0, c["top_p"] * 0.95), c["top_k"], presence=c["presence"],
                                    frequency=c["frequency"], repetition=c["repetition"])
                 for c in w.configs]]

    # Each set's call marshalled once (the C ABI call itself runs every step).
    launches = [sampler.prepare(sets[k][0], sets[k][2], tokens[k], counts=sets[k][1],
                                row_status=status[k], logprobs=L,
                                logprob_values=lpv[k] if L else None,
                                logprob_ids=lpi[k] if L else None) for k in range(nsets)]
    sid = stream.cuda_stream

    def step(i):
        if args.per_step_configs:
            sampler.set_configs(ctl_sets[i % 2], flags=w.flags, stream=sid)
        launches[i % nsets](sid)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for i in range(args.steps):
        step(args.warmup + i)
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(end)
    per_launch_s = ms / 1e3 / args.steps
    rows_per_s = w.rows * args.steps / (ms / 1e3)
    achieved = w.alg_bytes / per_launch_s / 1e9
    written = min(nsets, args.warmup + args.steps)
    bad = int((status[:written] != 0).sum())
    assert bad == 0, f"{bad} rows of {written} written sets reported errors"
    if args.per_step_configs:
        # Batch 0 again with the workload's own controls, for the parity check.
        sampler.set_configs(ctl_sets[0], flags=w.flags, stream=stream.cuda_stream)
        x, c, u = sets[0]
        sampler.sample(x, u, tokens[0], counts=c, row_status=status[0], logprobs=L,
                       logprob_values=lpv[0] if L else None, logprob_ids=lpi[0] if L else None,
                       stream=stream.cuda_stream)
        torch.cuda.synchronize()
    x0, c0, u0 = (t.cpu().numpy() for t in sets[0])
    c0 = c0.view("uint32")
    parity = oracle_parity(
        w, x0, c0, u0, tokens[0].cpu().numpy().view("uint32"), status[0].cpu().numpy(),
        (lpv[0].cpu().numpy(), lpi[0].cpu().numpy().view("uint32")) if L else None)

    traffic = None
    if args.config == 2 and TRAFFIC_FILE.exists():
        traffic = json.loads(TRAFFIC_FILE.read_text()).get("hbm_bytes_per_launch")

    line = {
        "metric": METRIC if args.config == 2 else
        f"sampled rows/sec @ vocab 151,936, batch {w.rows}; achieved HBM GB/s vs peak",
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
        "data": f"synthetic (device-generated config-{args.config} batches, rotated over "
                f"{nsets} distinct sets = {nsets * batch_bytes / 1e9:.2f} GB)",
        "config": {"workload": w.name + (", controls uploaded every step"
                                         if args.per_step_configs else ""),
                   "rows": w.rows, "vocab": VOCAB, "global_batch": w.rows,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "kernel": "fg::sample_rows_kernel",
                     "algorithmic_bytes_per_launch": w.alg_bytes,
                     "launch_us": round(per_launch_s * 1e6, 3)},
        "wall_s": round(wall, 3),
    }
    line["parity"] = parity
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(w, x0, c0, u0, args.cpu_seconds)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
