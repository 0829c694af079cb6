"""Synthetic inputs of the five BASELINE.json configs, built with the oracle's
Philox4x32-10 generators so CPU and GPU see identical bytes.  `rows` and `vocab`
can be reduced for oracle-speed parity tests; seeds are 1001..1005."""
from __future__ import annotations

import numpy as np

import oracle_ffi as O

V = 151_936


def cfg(temperature, top_p=1.0, top_k=1, presence=0.0, frequency=0.0, repetition=1.0):
    return dict(temperature=temperature, top_p=top_p, top_k=top_k, presence=presence,
                frequency=frequency, repetition=repetition)


def config1(rows=1, vocab=V):
    """Single row N(0,3^2); repetition 1.05 over 64 uniform history ids; greedy."""
    logits = O.gen_logits(rows, vocab, 0, 3.0, seed=1001, config_id=1)
    ids = O.gen_uniform_ids(rows, 64, vocab, 1001, 1)
    counts = O.build_counts(ids, vocab)
    configs = [cfg(0.0, 1.0, 1, repetition=1.05) for _ in range(rows)]
    return dict(logits=logits, counts=counts, configs=configs,
                uniforms=O.gen_uniforms(rows, 1001, 1), logprobs=0)


def config2(rows=64, vocab=V):
    """N(0,3^2) + 5 ids/row boosted by 8; Zipf(1.1) history of 1,024 -> presence 1.5,
    repetition 1.05; T 0.7, top-k 20, top-p 0.8."""
    logits = O.gen_logits(rows, vocab, 0, 3.0, seed=1002, config_id=2)
    boost = O.gen_uniform_ids(rows, 5, vocab, 1002, 22)
    for r in range(rows):
        logits[r, boost[r]] += np.float32(8.0)
    ids = O.gen_zipf_ids(rows, 1024, vocab, 1.1, 1002, 2)
    counts = O.build_counts(ids, vocab)
    configs = [cfg(0.7, 0.8, 20, presence=1.5, repetition=1.05) for _ in range(rows)]
    return dict(logits=logits, counts=counts, configs=configs,
                uniforms=O.gen_uniforms(rows, 1002, 2), logprobs=0)


def config3(rows=256, vocab=V):
    """2 * Student-t(3); Zipf history of 8,192 -> presence 0.5, frequency 0.3; T 1.0;
    top-p 0.95 over the whole vocabulary (top_k 0, extension)."""
    logits = O.gen_logits(rows, vocab, 1, 2.0, nu=3.0, seed=1003, config_id=3)
    ids = O.gen_zipf_ids(rows, 8192, vocab, 1.1, 1003, 3)
    counts = O.build_counts(ids, vocab)
    configs = [cfg(1.0, 0.95, 0, presence=0.5, frequency=0.3) for _ in range(rows)]
    return dict(logits=logits, counts=counts, configs=configs,
                uniforms=O.gen_uniforms(rows, 1003, 3), logprobs=0)


def config4(rows=128, vocab=V, sampled=True):
    """N(0,3^2) quantised to 0.25 in [-16,16], one id/row = +20; greedy or
    top-k 50 / top-p 0.9; rows 0..rows/2-1 repetition 1.1 over 256 uniform ids."""
    logits = O.gen_logits(rows, vocab, 2, 3.0, seed=1004, config_id=4)
    spike = O.gen_uniform_ids(rows, 1, vocab, 1004, 44)
    for r in range(rows):
        logits[r, spike[r, 0]] = np.float32(20.0)
    ids = O.gen_uniform_ids(rows, 256, vocab, 1004, 4)
    counts = O.build_counts(ids, vocab)
    half = rows // 2
    configs = []
    for r in range(rows):
        rep = 1.1 if r < half else 1.0
        configs.append(cfg(0.8, 0.9, 50, repetition=rep) if sampled else cfg(0.0, 1.0, 1, repetition=rep))
    return dict(logits=logits, counts=counts, configs=configs,
                uniforms=O.gen_uniforms(rows, 1004, 4), logprobs=0)


def config5(rows=1024, vocab=V):
    """Rows alternate N(0,2^2)/N(0,6^2); Zipf history of 32,768 -> presence 1.0,
    frequency 0.2, repetition 1.05; T 0.6, top-k 64, top-p 0.95; top-20 log-probs."""
    logits = O.gen_logits(rows, vocab, 3, 2.0, sigma2=6.0, seed=1005, config_id=5)
    ids = O.gen_zipf_ids(rows, 32768, vocab, 1.1, 1005, 5)
    counts = O.build_counts(ids, vocab)
    configs = [cfg(0.6, 0.95, 64, presence=1.0, frequency=0.2, repetition=1.05)
               for _ in range(rows)]
    return dict(logits=logits, counts=counts, configs=configs,
                uniforms=O.gen_uniforms(rows, 1005, 5), logprobs=20)


def oracle_run(w, logprobs=None, want_penalised=False, threads=4):
    return O.sample_rows(w["configs"], w["logits"], w["uniforms"], counts=w["counts"],
                         logprobs=w["logprobs"] if logprobs is None else logprobs,
                         want_penalised=want_penalised, threads=threads)
