"""GPU parity over seeded random batches: controls, geometry and data drawn
per case (greedy, top-k 1-64, whole-row nucleus and log-probs mixed or alone;
penalties on some rows; ties, plateaus and non-finite values; vocabularies
that split unevenly; 1-64 workgroups per row and both row hand-offs), each
against the C oracle on the same inputs at the north-star bar (ids exact
except within 1e-6 of a boundary; 1e-11 for whole-row nucleus rows, whose
masses are summed differently).  The cases are fixed by their seeds."""
import numpy as np
import pytest

import fg_hip
import workloads as W
from test_gpu_sampler import BOUNDARY, NUC_BOUNDARY, check, run_hip

pytestmark = pytest.mark.gpu


def random_case(seed):
    rng = np.random.default_rng(seed)
    rows = int(rng.choice([1, 2, 5, 8, 16, 24]))
    vocab = int(rng.choice([97, 1000, 4099, 20_000, 65_537]))
    kind = rng.choice(["topk", "greedy", "mixed", "nucleus", "logprobs"])
    logits = rng.normal(0, rng.choice([0.5, 3.0, 8.0]), (rows, vocab)).astype(np.float32)
    for r in range(rows):
        shape = rng.integers(0, 6)
        if shape == 1:  # quantised: many exact ties
            logits[r] = np.round(logits[r] * 4) / 4
        elif shape == 2:  # a plateau at the top
            logits[r, rng.integers(0, vocab, 40)] = logits[r].max() + 1.0
        elif shape == 3:  # a few non-finite values
            logits[r, rng.integers(0, vocab, 3)] = rng.choice([np.nan, np.inf, -np.inf])
        elif shape == 4:  # one dominant value
            logits[r, rng.integers(0, vocab)] = 40.0
    counts = np.zeros((rows, vocab), dtype=np.uint32)
    configs = []
    for r in range(rows):
        pen = rng.random() < 0.5
        pres, freq, rep = ((float(rng.choice([0.0, 0.5, 1.5])), float(rng.choice([0.0, 0.2])),
                            float(rng.choice([1.0, 1.05, 1.3]))) if pen else (0.0, 0.0, 1.0))
        if pen:
            ids = rng.integers(0, vocab, int(rng.integers(1, 300)))
            np.add.at(counts[r], ids, 1)
        k = {"topk": int(rng.integers(1, 65)), "greedy": 0, "nucleus": -1,
             "logprobs": int(rng.integers(1, 65)),
             "mixed": int(rng.choice([0, 1, 20, 64, -1]))}[kind]
        if k == 0:
            configs.append(W.cfg(0.0, 1.0, 1, pres, freq, rep))
        elif k == -1:
            configs.append(W.cfg(float(rng.choice([0.6, 1.0])), float(rng.choice([0.5, 0.95])),
                                 0, pres, freq, rep))
        else:
            configs.append(W.cfg(float(rng.choice([0.3, 0.7, 1.2])),
                                 float(rng.choice([0.5, 0.8, 1.0])), k, pres, freq, rep))
    w = dict(logits=logits, counts=counts, configs=configs,
             uniforms=rng.random(rows).astype(np.float32),
             logprobs=int(rng.integers(1, 33)) if kind == "logprobs" else 0)
    groups = int(rng.choice([0, 8, 64, 256, 1024]))  # 0: the geometry rule
    finisher = str(rng.choice(["-", "0", "1", "2"]))
    return w, groups, finisher


@pytest.mark.parametrize("seed", list(range(160)))
def test_random_batch_matches_oracle(dev, monkeypatch, seed):
    w, groups, finisher = random_case(1000 + seed)
    if groups:
        monkeypatch.setenv("FG_HIP_TARGET_GROUPS", str(groups))
    if finisher != "-":
        monkeypatch.setenv("FG_HIP_FINISHER", finisher)
    nuc = any(c["top_k"] == 0 and c["temperature"] > 0.0 for c in w["configs"])
    flags = fg_hip.ALLOW_FULL_VOCAB if nuc else 0
    rows = len(w["configs"])
    s = fg_hip.HipSampler(w["logits"].shape[1], rows)
    for call in range(2):  # twice on one sampler: the workspace is left as found
        check(w, run_hip(w, dev, flags=flags, sampler=s), W.oracle_run(w),
              f"seed {seed} groups {groups} finisher {finisher} call {call}",
              NUC_BOUNDARY if nuc else BOUNDARY)
