"""GPU parity: the HIP batched sampler (C ABI fg_sampler_hip_sample) against the
CPU oracle on identical inputs and identical per-row uniforms.

Bar: token ids bit-exact, except where the oracle's
f64 running sums come within 1e-6 (relative) of a top-p or draw boundary;
penalised logits within 1e-6 relative (the C rounding is reproduced exactly, so
the check is bit-exact); log-probs within 1e-5 absolute.
"""
import numpy as np
import pytest

import fg_hip
import workloads as W

pytestmark = pytest.mark.gpu

BOUNDARY = 1e-6
LP_TOL = 1e-5
# Whole-row nucleus masses are summed with an f64 exp of a few ulp: tokens
# must match the oracle except where its sums come within 1e-11 of a
# boundary (1e-6, would excuse most deep cuts, whose
# steps are ~1e-5 of the mass each).
NUC_BOUNDARY = 1e-11


def to_dev(a, dev):
    import torch
    if a.dtype == np.uint32:
        return torch.from_numpy(a.view(np.int32)).to(dev)
    return torch.from_numpy(a).to(dev)


def run_hip(w, dev, logprobs=None, penalised=False, flags=0, sampler=None, counts=True):
    import torch
    logits = w["logits"]
    rows, vocab = logits.shape
    L = w["logprobs"] if logprobs is None else logprobs
    s = sampler or fg_hip.HipSampler(vocab, rows)
    s.set_configs([fg_hip.make_config(c["temperature"], c["top_p"], c["top_k"], c["presence"],
                                      c["frequency"], c["repetition"]) for c in w["configs"]],
                  flags=flags)
    d_logits = to_dev(logits, dev)
    d_counts = to_dev(w["counts"], dev) if counts else None
    d_u = to_dev(w["uniforms"], dev)
    tok = torch.empty(rows, dtype=torch.int32, device=dev)
    tl = torch.empty(rows, dtype=torch.float32, device=dev)
    st = torch.empty(rows, dtype=torch.int32, device=dev)
    pen = torch.empty((rows, vocab), dtype=torch.float32, device=dev) if penalised else None
    lpv = torch.empty((rows, max(L, 1)), dtype=torch.float32, device=dev)
    lpi = torch.empty((rows, max(L, 1)), dtype=torch.int32, device=dev)
    s.sample(d_logits, d_u, tok, counts=d_counts, token_logits=tl, row_status=st, penalised=pen,
             logprobs=L, logprob_values=lpv if L else None, logprob_ids=lpi if L else None)
    torch.cuda.synchronize()
    out = dict(token=tok.cpu().numpy().view(np.uint32), logit=tl.cpu().numpy(),
               status=st.cpu().numpy())
    if penalised:
        out["penalised"] = pen.cpu().numpy()
    if L:
        out["lp_values"] = lpv.cpu().numpy()[:, :L]
        out["lp_ids"] = lpi.cpu().numpy().view(np.uint32)[:, :L]
    return out


def check(w, got, ref, name, boundary=BOUNDARY):
    st_ok = np.array_equal(got["status"], ref["status"])
    assert st_ok, f"{name}: status {got['status']} vs {ref['status']}"
    ok = ref["status"] == 0
    same = got["token"] == ref["token"]
    near = ref["margin"] < boundary
    bad = ok & ~same & ~near
    assert not bad.any(), (
        f"{name}: rows {np.nonzero(bad)[0][:10]} token {got['token'][bad][:10]} "
        f"vs oracle {ref['token'][bad][:10]} (margin {ref['margin'][bad][:10]})")
    exact = ok & same
    assert np.array_equal(got["logit"][exact].view(np.uint32), ref["logit"][exact].view(np.uint32)), \
        f"{name}: token logits differ"
    if "lp_values" in ref:
        assert np.array_equal(got["lp_ids"], ref["lp_ids"]), f"{name}: log-prob ids differ"
        fin = np.isfinite(ref["lp_values"])
        assert np.array_equal(fin, np.isfinite(got["lp_values"]))
        err = np.abs(got["lp_values"][fin].astype(np.float64) - ref["lp_values"][fin])
        assert err.max(initial=0.0) <= LP_TOL, f"{name}: log-prob error {err.max()}"
    return int(near.sum())


def test_config1_greedy_repetition(dev):
    w = W.config1()
    check(w, run_hip(w, dev), W.oracle_run(w), "config1")


def test_config2_north_star(dev):
    w = W.config2()
    got = run_hip(w, dev, penalised=True)
    ref = W.oracle_run(w, want_penalised=True)
    check(w, got, ref, "config2")
    assert np.array_equal(got["penalised"].view(np.uint32), ref["penalised"].view(np.uint32))


def test_config2_repeated_launches(dev):
    """The row counters and thresholds reset themselves: three launches in a row
    on one sampler, the middle one with fewer rows, all match."""
    w = W.config2(rows=48)
    s = fg_hip.HipSampler(W.V, 48)
    ref = W.oracle_run(w)
    check(w, run_hip(w, dev, sampler=s), ref, "launch 1")
    small = {k: (v[:17] if k in ("logits", "counts", "uniforms", "configs") else v)
             for k, v in w.items()}
    check(small, run_hip(small, dev, sampler=s), W.oracle_run(small), "launch 2")
    check(w, run_hip(w, dev, sampler=s), ref, "launch 3")


@pytest.mark.parametrize("sampled", [False, True])
def test_config4_ties(dev, sampled):
    w = W.config4(sampled=sampled)
    check(w, run_hip(w, dev), W.oracle_run(w), f"config4 sampled={sampled}")


def cores():
    import os
    return len(os.sched_getaffinity(0))


def test_config5_logprobs(dev):
    w = W.config5(rows=64)
    check(w, run_hip(w, dev), W.oracle_run(w, threads=cores()), "config5")


def test_config5_full_batch(dev):
    """Config 5 at its stated batch: 1,024 rows, which the launch rule runs at
    one workgroup per row (the row merged in LDS, no cross-workgroup
    hand-off), with top-k 64 and 20 log-probs."""
    assert fg_hip.plan(W.V, 1024).chunks == 1
    w = W.config5()
    check(w, run_hip(w, dev), W.oracle_run(w, threads=cores()), "config5 1024 rows")


@pytest.mark.parametrize("k,logprobs", [(20, 0), (64, 20), (0, 0)])
def test_one_chunk_rows_full_vocab(dev, monkeypatch, k, logprobs):
    """One workgroup per row at V=151,936 forced on a 64-row batch
    (FG_HIP_TARGET_GROUPS=64): top-k 20, top-k 64 with log-probs and the
    whole-row nucleus, all through the single-chunk finish."""
    monkeypatch.setenv("FG_HIP_TARGET_GROUPS", "64")
    assert fg_hip.plan(W.V, 64).chunks == 1
    w = W.config5(rows=64)
    w["logprobs"] = logprobs
    flags = 0
    if k == 0:
        w = W.config3(rows=64)
        flags = fg_hip.ALLOW_FULL_VOCAB
    else:
        w["configs"] = [dict(c, top_k=k) for c in w["configs"]]
    check(w, run_hip(w, dev, flags=flags), W.oracle_run(w, threads=cores()),
          f"one chunk k={k}", NUC_BOUNDARY if k == 0 else BOUNDARY)


def test_owner_loop_controls_change_every_call(dev):
    """The output owner's loop: every row's controls (temperature, top-p,
    top-k, penalties, greedy rows) and uniforms change on every call, with
    set_configs before each sample and no synchronisation anywhere in the
    loop; each call's results match the oracle run with that call's
    controls."""
    import torch
    rows, calls = 16, 10
    base = W.config2(rows=rows)
    rng = np.random.default_rng(7)
    s = fg_hip.HipSampler(W.V, rows)
    d_logits = to_dev(base["logits"], dev)
    d_counts = to_dev(base["counts"], dev)
    plans = []
    toks = torch.full((calls, rows), -1, dtype=torch.int32, device=dev)
    tls = torch.zeros((calls, rows), dtype=torch.float32, device=dev)
    sts = torch.full((calls, rows), -1, dtype=torch.int32, device=dev)
    d_us = []
    torch.cuda.synchronize()
    for i in range(calls):
        cfgs = []
        for r in range(rows):
            if rng.random() < 0.2:
                cfgs.append(W.cfg(0.0, 1.0, 1, repetition=float(rng.choice([1.0, 1.1]))))
            else:
                cfgs.append(W.cfg(float(rng.uniform(0.2, 1.5)), float(rng.uniform(0.3, 1.0)),
                                  int(rng.integers(1, 65)), presence=float(rng.uniform(0, 2)),
                                  frequency=float(rng.uniform(0, 1)),
                                  repetition=float(rng.uniform(0.9, 1.2))))
        u = rng.random(rows).astype(np.float32)
        d_u = torch.from_numpy(u).to(dev, non_blocking=False)
        d_us.append(d_u)
        s.set_configs([fg_hip.make_config(c["temperature"], c["top_p"], c["top_k"], c["presence"],
                                          c["frequency"], c["repetition"]) for c in cfgs])
        s.sample(d_logits, d_u, toks[i], counts=d_counts, token_logits=tls[i], row_status=sts[i])
        plans.append((cfgs, u))
    torch.cuda.synchronize()
    for i, (cfgs, u) in enumerate(plans):
        w = dict(base, configs=cfgs, uniforms=u)
        got = dict(token=toks[i].cpu().numpy().view(np.uint32), logit=tls[i].cpu().numpy(),
                   status=sts[i].cpu().numpy())
        check(w, got, W.oracle_run(w, threads=cores()), f"owner call {i}")


def test_controls_reach_the_table_for_later_calls(dev):
    """set_configs launches nothing: up to 64 configured rows travel in the
    next sample's arguments (which also writes them to the device table),
    more go by fill kernels first.  A smaller batch after set_configs, then
    the full batch again with no set_configs in between (read from the
    table), then 80 rows (fill kernels): each call matches the oracle with
    the controls last set."""
    for rows in (64, 80):
        w = W.config2(rows=rows)
        for r in range(0, rows, 5):
            w["configs"][r] = W.cfg(0.0, 1.0, 1, repetition=1.1)  # greedy rows mixed in
        s = fg_hip.HipSampler(W.V, rows)
        s.set_configs([fg_hip.make_config(c["temperature"], c["top_p"], c["top_k"], c["presence"],
                                          c["frequency"], c["repetition"]) for c in w["configs"]])
        half = dict(w, logits=w["logits"][:16], counts=w["counts"][:16],
                    configs=w["configs"][:16], uniforms=w["uniforms"][:16])
        check(half, run_hip_configured(half, dev, s), W.oracle_run(half), f"{rows}: first 16 rows")
        check(w, run_hip_configured(w, dev, s), W.oracle_run(w), f"{rows}: all rows, from the table")


def run_hip_configured(w, dev, s):
    """run_hip on a sampler whose controls are already set (no set_configs)."""
    import torch
    rows = w["logits"].shape[0]
    tok = torch.empty(rows, dtype=torch.int32, device=dev)
    tl = torch.empty(rows, dtype=torch.float32, device=dev)
    st = torch.empty(rows, dtype=torch.int32, device=dev)
    s.sample(to_dev(np.ascontiguousarray(w["logits"]), dev), to_dev(w["uniforms"], dev), tok,
             counts=to_dev(np.ascontiguousarray(w["counts"]), dev), token_logits=tl, row_status=st)
    torch.cuda.synchronize()
    return dict(token=tok.cpu().numpy().view(np.uint32), logit=tl.cpu().numpy(),
                status=st.cpu().numpy())


def test_mixed_rows_and_greedy_logprobs(dev):
    """Greedy, sampled and unpenalised rows in one batch, with log-probs."""
    w = W.config2(rows=12)
    for r in range(0, 12, 3):
        w["configs"][r] = W.cfg(0.0, 1.0, 1, presence=0.5 if r % 2 else 0.0)
    w["configs"][4] = W.cfg(1.3, 0.5, 64)
    w["configs"][5] = W.cfg(0.2, 1.0, 1)
    w["logprobs"] = 8
    check(w, run_hip(w, dev), W.oracle_run(w), "mixed")


@pytest.mark.parametrize("vocab", [1, 3, 5, 63, 64, 1000, 1001, 4097, 65537])
def test_small_and_ragged_vocab(dev, vocab):
    w = W.config2(rows=5, vocab=vocab)
    w["configs"][0] = W.cfg(0.0, 1.0, 1)
    w["logprobs"] = 4
    check(w, run_hip(w, dev), W.oracle_run(w), f"vocab {vocab}")


def test_non_finite_and_ties(dev):
    rng = np.random.default_rng(7)
    vocab = 20_000
    rows = 10
    logits = rng.normal(0, 2, (rows, vocab)).astype(np.float32)
    logits[0, 777] = np.nan                      # greedy: non-finite wins -> error
    logits[1, :] = 1.5                           # all equal: lowest ids win
    logits[2, ::2] = np.inf                      # half +inf: excluded by top-k
    logits[3, :] = np.nan
    logits[3, [5, 900, 19_999]] = [1.0, 2.0, 2.0]  # only 3 finite, k=20
    logits[4, :] = 0.0
    logits[4, ::3] = -0.0                        # +0 ranks above -0 in the key order
    logits[5, :] = np.nan                        # no finite candidate -> error
    logits[6, 100] = np.float32(3e38)            # large values
    logits[6, 101] = np.float32(3e38)
    logits[7, :] = -np.inf
    logits[7, 42] = -1e30
    counts = np.zeros((rows, vocab), dtype=np.uint32)
    counts[:, 900] = 3
    counts[:, 100] = 0xFFFFFFFF
    configs = [W.cfg(0.0, 1.0, 1), W.cfg(0.5, 0.9, 20), W.cfg(0.5, 0.9, 20),
               W.cfg(0.5, 0.9, 20, presence=0.25), W.cfg(0.5, 1.0, 20),
               W.cfg(0.5, 1.0, 20), W.cfg(1.0, 0.5, 2, frequency=0.5), W.cfg(0.0, 1.0, 1),
               W.cfg(0.0, 1.0, 1, repetition=1.2), W.cfg(0.0, 1.0, 1)]
    logits[8, :] = np.float32(2.0)
    logits[9, :] = np.float32(-2.0)
    logits[9, 12] = np.inf
    w = dict(logits=logits, counts=counts, configs=configs,
             uniforms=np.linspace(0.05, 0.95, rows).astype(np.float32), logprobs=5)
    check(w, run_hip(w, dev), W.oracle_run(w), "non-finite")


def test_uniform_edges(dev):
    w = W.config2(rows=6, vocab=5000)
    w["uniforms"] = np.array([0.0, -1.0, np.nan, 1.0, 2.0, np.float32(0.99999994)],
                             dtype=np.float32)
    check(w, run_hip(w, dev), W.oracle_run(w), "uniform edges")


def test_strided_rows_and_no_counts(dev):
    import torch
    w = W.config2(rows=8, vocab=3001)
    ref = W.oracle_run(dict(w, counts=np.zeros_like(w["counts"])))
    s = fg_hip.HipSampler(3001, 8)
    s.set_configs([fg_hip.make_config(**{"temperature": c["temperature"], "top_p": c["top_p"],
                                         "top_k": c["top_k"]}) for c in w["configs"]])
    big = np.zeros((8, 3007), dtype=np.float32)
    big[:, :3001] = w["logits"]
    d = to_dev(big, dev)
    tok = torch.empty(8, dtype=torch.int32, device=dev)
    st = torch.empty(8, dtype=torch.int32, device=dev)
    s.sample(d, to_dev(w["uniforms"], dev), tok, row_status=st, logits_stride=3007)
    torch.cuda.synchronize()
    assert np.array_equal(st.cpu().numpy(), ref["status"])
    got = tok.cpu().numpy().view(np.uint32)
    near = ref["margin"] < BOUNDARY
    assert np.all((got == ref["token"]) | near)


def test_argument_errors(dev):
    import torch
    s = fg_hip.HipSampler(100, 4)
    with pytest.raises(fg_hip.FgStatusError) as e:
        s.set_configs([fg_hip.make_config(top_k=65)])
    assert e.value.code == fg_hip.FG_ERR_ARGUMENT
    with pytest.raises(fg_hip.FgStatusError):
        s.set_configs([fg_hip.make_config(min_p=0.1)])
    with pytest.raises(fg_hip.FgStatusError):
        s.set_configs([fg_hip.make_config(top_k=0)])
    s.set_configs([fg_hip.make_config(top_k=0)], flags=fg_hip.ALLOW_FULL_VOCAB)
    with pytest.raises(fg_hip.FgStatusError):
        s.set_configs([fg_hip.make_config()], flags=4)
    s.set_configs([fg_hip.make_config()] * 4)
    x = torch.zeros((4, 100), device=dev)
    u = torch.zeros(4, device=dev)
    t = torch.zeros(4, dtype=torch.int32, device=dev)
    with pytest.raises(fg_hip.FgStatusError):
        s.sample(x, u, t, rows=5)
    with pytest.raises(fg_hip.FgStatusError):
        s.sample(x, u, t, logits_stride=99)
    with pytest.raises(fg_hip.FgStatusError):
        s.sample(x, u, t, logprobs=65, logprob_values=x, logprob_ids=t)


def test_history_increment(dev):
    import torch
    vocab, rows = 1000, 4
    s = fg_hip.HipSampler(vocab, rows)
    s.set_configs([fg_hip.make_config(presence=1.0), fg_hip.make_config(),
                   fg_hip.make_config(repetition=1.1), fg_hip.make_config(frequency=0.1)])
    counts = torch.zeros((rows, vocab), dtype=torch.int32, device=dev)
    counts[3, 9] = -1  # UINT32_MAX saturates
    tokens = torch.tensor([5, 6, 7, 9], dtype=torch.int32, device=dev)
    status = torch.tensor([0, 0, 4, 0], dtype=torch.int32, device=dev)
    s.history_increment(counts, tokens, row_status=status)
    torch.cuda.synchronize()
    c = counts.cpu().numpy().view(np.uint32)
    assert c[0, 5] == 1 and c[1, 6] == 0 and c[2, 7] == 0 and c[3, 9] == 0xFFFFFFFF
    assert c.sum(dtype=np.uint64) == 1 + 0xFFFFFFFF


def test_config3_whole_row_nucleus(dev):
    w = W.config3(rows=64)
    ref = W.oracle_run(w, threads=cores())
    assert (ref["cutoff"] <= 64).all()
    check(w, run_hip(w, dev, flags=fg_hip.ALLOW_FULL_VOCAB), ref, "config3", NUC_BOUNDARY)


def test_config3_full_batch(dev):
    """Config 3 at its stated batch: 256 rows, three unpaired chunks per row
    (the nucleus launch rule)."""
    g = fg_hip.plan(W.V, 256, fg_hip.ROWS_NUCLEUS)
    assert (g.chunks, g.split) == (3, 3)
    w = W.config3()
    check(w, run_hip(w, dev, flags=fg_hip.ALLOW_FULL_VOCAB), W.oracle_run(w, threads=cores()),
          "config3 256 rows", NUC_BOUNDARY)


def test_nucleus_cut_depths(dev):
    """N(0, s^2) rows at T 1: s = 12 and 8 cut inside the 64 best (fused
    pass), s = 1 thousands deep (deep-row kernel); rows with 100, 40 and 30
    finite logits."""
    import oracle_ffi as O
    vocab = 151_936
    logits = np.concatenate([O.gen_logits(4, vocab, 0, 12.0, seed=7, config_id=31),
                             O.gen_logits(4, vocab, 0, 8.0, seed=7, config_id=32),
                             O.gen_logits(4, vocab, 0, 1.0, seed=7, config_id=33)])
    rows = logits.shape[0]
    logits[3, 100:] = np.nan
    logits[7, 40:] = -np.inf
    logits[11, 30:] = np.nan
    configs = [W.cfg(1.0, p, 0, presence=0.3) for p in (0.5, 0.9, 0.95, 0.99)] * 3
    counts = np.zeros((rows, vocab), dtype=np.uint32)
    counts[:, ::1000] = 2
    w = dict(logits=logits, counts=counts, configs=configs,
             uniforms=np.linspace(0.02, 0.98, rows).astype(np.float32), logprobs=0)
    ref = W.oracle_run(w)
    assert (ref["cutoff"] <= 64).sum() >= 6 and (ref["cutoff"] > 1000).sum() >= 2
    check(w, run_hip(w, dev, flags=fg_hip.ALLOW_FULL_VOCAB), ref, "nucleus depths", NUC_BOUNDARY)


def test_nucleus_deep_rows(dev):
    """Deep cuts: flat rows, whole-row ties (cut and draw inside one value),
    +0 / -0 mixes, top_p 1 and 0.9999 (cut in the far tail), tempered draws,
    penalties, and a uniform at each end."""
    rng = np.random.default_rng(11)
    vocab = 151_936
    rows = 12
    logits = rng.normal(0, 1, (rows, vocab)).astype(np.float32)
    logits[1, :] = 0.5                               # all tied
    logits[2, :] = 0.0
    logits[2, ::2] = -0.0                            # zeros of both signs
    logits[3, :] = np.round(rng.normal(0, 1, vocab) * 4) / 4   # many ties
    logits[4, :] = rng.normal(0, 0.01, vocab)        # nearly flat
    logits[5, :] = rng.normal(0, 6, vocab)           # wide
    logits[6, : vocab // 2] = np.nan
    logits[7, :] = np.float32(-1e30)
    logits[7, 5::7] = np.float32(-1e30) + 1e24
    configs = [W.cfg(1.0, 0.9, 0), W.cfg(1.0, 0.37, 0), W.cfg(0.8, 0.5, 0, presence=0.0),
               W.cfg(1.5, 0.95, 0), W.cfg(0.2, 0.9, 0), W.cfg(2.0, 0.999, 0),
               W.cfg(1.0, 0.7, 0, presence=1.0, frequency=0.5), W.cfg(1.0, 0.6, 0),
               W.cfg(1.0, 1.0, 0), W.cfg(0.7, 0.9999, 0), W.cfg(3.0, 0.8, 0, repetition=1.3),
               W.cfg(1.0, 0.9, 0, presence=-0.5)]
    counts = np.zeros((rows, vocab), dtype=np.uint32)
    hot = rng.integers(0, vocab, (rows, 5000))
    np.add.at(counts, (np.repeat(np.arange(rows), 5000), hot.ravel()), 1)
    u = rng.random(rows).astype(np.float32)
    u[0], u[8] = 0.0, np.float32(0.99999994)
    w = dict(logits=logits, counts=counts, configs=configs, uniforms=u, logprobs=3)
    ref = W.oracle_run(w)
    assert (ref["cutoff"] > 64).sum() >= 9
    check(w, run_hip(w, dev, flags=fg_hip.ALLOW_FULL_VOCAB), ref, "deep nucleus", NUC_BOUNDARY)


@pytest.mark.parametrize("vocab", [65, 100, 4097, 10_000])
def test_nucleus_small_vocab(dev, vocab):
    rng = np.random.default_rng(vocab)
    rows = 6
    logits = rng.normal(0, 0.5, (rows, vocab)).astype(np.float32)
    logits[1, :] = 1.0
    configs = [W.cfg(1.0, p, 0) for p in (0.3, 0.6, 0.9, 0.99, 1.0, 0.5)]
    w = dict(logits=logits, counts=np.zeros((rows, vocab), np.uint32), configs=configs,
             uniforms=rng.random(rows).astype(np.float32), logprobs=0)
    check(w, run_hip(w, dev, flags=fg_hip.ALLOW_FULL_VOCAB), W.oracle_run(w), f"nucleus {vocab}",
          NUC_BOUNDARY)


def test_nucleus_mixed_with_top_k_rows_and_logprobs(dev):
    w = W.config3(rows=16, vocab=50_000)
    for r in range(0, 16, 4):
        w["configs"][r] = W.cfg(0.7, 0.8, 20, presence=1.5, repetition=1.05)
    w["configs"][1] = W.cfg(0.0, 1.0, 1)
    w["configs"][2] = W.cfg(1.0, 0.9, 0)
    w["logits"][2] = np.random.default_rng(3).normal(0, 1, 50_000).astype(np.float32)
    w["logprobs"] = 5
    ref = W.oracle_run(w)
    assert ref["cutoff"][2] > 64
    check(w, run_hip(w, dev, flags=fg_hip.ALLOW_FULL_VOCAB), ref, "nucleus mixed", NUC_BOUNDARY)


@pytest.mark.parametrize("k,logprobs", [(20, 0), (64, 0), (20, 40), (40, 0), (5, 0), (0, 0)])
def test_speculative_filter_rescans(dev, k, logprobs):
    """Rows built so that a wave's early elements hold most of the row's best
    values: the speculative stream filter then skips elements that belong in
    the row's top-k (or a nucleus row's 64 best), and the merge must read
    those slices again.  Also
    ascending, descending and tied rows, a row with few finite values, and
    values just below the speculative filter.  Exact against the oracle."""
    rng = np.random.default_rng(17 + k)
    rows, vocab = 12, W.V
    logits = rng.normal(0, 1, (rows, vocab)).astype(np.float32)
    logits[0, :600] = 50 + rng.normal(0, 1, 600)                 # top values at the row start
    logits[1] = np.linspace(-5, 5, vocab, dtype=np.float32)       # ascending
    logits[2] = np.linspace(5, -5, vocab, dtype=np.float32)       # descending
    logits[3, :] = 1.0                                            # all tied
    logits[3, 5000:5100] = 2.0
    logits[4, :] = -np.inf                                        # few finite values
    logits[4, rng.choice(vocab, 90, replace=False)] = rng.normal(0, 1, 90)
    logits[5, 37984:37984 + 1500] = 20 + rng.normal(0, 1, 1500)   # one slice holds the top
    logits[6, 0:300:3] = 30.0                                     # tied top values, spread out
    logits[7, 151_000:] = 40 + rng.normal(0, 1, vocab - 151_000)  # top values in the row tail
    for r in (8, 9):                                              # clustered per 1024-element step
        for b in range(0, vocab, 4096):
            logits[r, b:b + 8] = 10 + rng.normal(0, 0.1, 8)
    logits[10, :64 * 16] = 9.0 + np.arange(1024, dtype=np.float32) * 1e-3  # one value per lane
    counts = np.zeros((rows, vocab), dtype=np.uint32)
    counts[11, :300] = rng.integers(1, 5, 300)                    # penalties on the top values
    logits[11, :300] = 60.0
    # k == 0: the whole-row nucleus, whose list of the 64 best speculates too.
    configs = [W.cfg(0.8, 0.9 if k else 0.2, k, presence=0.4 if r == 11 else 0.0)
               for r in range(rows)]
    w = dict(logits=logits, counts=counts, configs=configs,
             uniforms=rng.random(rows).astype(np.float32), logprobs=logprobs)
    if k:
        check(w, run_hip(w, dev), W.oracle_run(w), f"speculation k={k} L={logprobs}")
    else:
        check(w, run_hip(w, dev, flags=fg_hip.ALLOW_FULL_VOCAB), W.oracle_run(w),
              "speculation nucleus", NUC_BOUNDARY)


@pytest.mark.parametrize("groups,share,k", [(32, 650, 20), (32, 650, 64), (32, 650, 0),
                                            (128, 500, 20), (128, 600, 64), (128, 560, 0)])
def test_paired_layout_shares(dev, monkeypatch, groups, share, k):
    """The paired layout (a row's first chunks in the grid's first half, with
    a larger share of the row, the rest in its second half): 16 rows, 2 or 8
    chunks per row, uneven slices; rows whose best values sit at slice
    edges, in one slice or in the row tail, and speculating lists that must
    rescan.  Exact against the oracle."""
    monkeypatch.setenv("FG_HIP_TARGET_GROUPS", str(groups))
    monkeypatch.setenv("FG_HIP_FRONT_SHARE", str(share))
    monkeypatch.setenv("FG_HIP_PAIRED", "1")  # row 7's penalties would keep row-major halves
    rng = np.random.default_rng(groups + share + k)
    rows, vocab = 16, W.V
    logits = rng.normal(0, 1, (rows, vocab)).astype(np.float32)
    logits[0, :600] = 50 + rng.normal(0, 1, 600)                  # top values at the row start
    logits[1] = np.linspace(-5, 5, vocab, dtype=np.float32)        # ascending
    logits[2, 75_000:80_000] = 20 + rng.normal(0, 1, 5000)         # across the halves' boundary
    logits[3, 151_000:] = 40 + rng.normal(0, 1, vocab - 151_000)   # the row tail
    logits[4, :] = 1.0                                             # tied, a few higher
    logits[4, 98_000:98_100] = 2.0
    for r in (5, 6):                                               # one value per 4096 block
        logits[r, ::4096] = 10 + rng.normal(0, 0.1, len(range(0, vocab, 4096)))
    counts = np.zeros((rows, vocab), dtype=np.uint32)
    counts[7, :300] = rng.integers(1, 5, 300)
    logits[7, :300] = 60.0
    configs = [W.cfg(0.8, 0.9 if k else 0.3, k, presence=0.4 if r == 7 else 0.0)
               for r in range(rows)]
    w = dict(logits=logits, counts=counts, configs=configs,
             uniforms=rng.random(rows).astype(np.float32), logprobs=0)
    if k:
        check(w, run_hip(w, dev), W.oracle_run(w), f"paired groups={groups} share={share} k={k}")
    else:
        check(w, run_hip(w, dev, flags=fg_hip.ALLOW_FULL_VOCAB), W.oracle_run(w),
              f"paired nucleus groups={groups} share={share}", NUC_BOUNDARY)


@pytest.mark.parametrize("groups,finisher,k", [(32, "1", 20), (32, "2", 32), (64, "3", 1),
                                               (128, "1", 20), (128, "6", 32), (128, "8", 7),
                                               (128, "0", 20), (256, "1", 20), (256, "1", 32),
                                               (32, "2", 33), (64, "4", 50), (128, "7", 64),
                                               (128, "1", 50)])
def test_finisher_rows(dev, monkeypatch, groups, finisher, k):
    """The finisher hand-off (one chunk of each row reads the others' tagged
    lists; FG_HIP_FINISHER=c+1 picks chunk c, 0 the last-arriver hand-off):
    16 rows over 2, 4 or 8 chunks, lists of 1-32 (two a register in the
    finisher) and of 33-64 (a position per lane), finishing chunks whose list
    sits in the low or the high (reversed) lanes, top values at slice edges and in one
    slice (16 chunks: more than the finisher takes, so the last-arriver
    hand-off runs, with the workgroups' rank merges); three calls on one sampler with new inputs each (the finisher
    clears the lists it reads, so a call sees none of the last one's).
    Exact against the oracle."""
    monkeypatch.setenv("FG_HIP_TARGET_GROUPS", str(groups))
    monkeypatch.setenv("FG_HIP_FINISHER", finisher)
    rows, vocab = 16, W.V
    s = fg_hip.HipSampler(vocab, rows)
    for call in range(3):
        rng = np.random.default_rng(groups * 10 + int(finisher) + 100 * call + k)
        logits = rng.normal(0, 1, (rows, vocab)).astype(np.float32)
        logits[0, :600] = 50 + rng.normal(0, 1, 600)
        logits[1] = np.linspace(-5, 5, vocab, dtype=np.float32)
        logits[2, 75_000:80_000] = 20 + rng.normal(0, 1, 5000)
        logits[3, 151_000:] = 40 + rng.normal(0, 1, vocab - 151_000)
        logits[4, :] = 1.0
        logits[4, 98_000:98_100] = 2.0
        counts = np.zeros((rows, vocab), dtype=np.uint32)
        counts[7, :300] = rng.integers(1, 5, 300)
        logits[7, :300] = 60.0
        configs = [W.cfg(0.8, 0.9, k, presence=0.4 if r == 7 else 0.0) for r in range(rows)]
        w = dict(logits=logits, counts=counts, configs=configs,
                 uniforms=rng.random(rows).astype(np.float32), logprobs=0)
        check(w, run_hip(w, dev, sampler=s), W.oracle_run(w),
              f"finisher groups={groups} finisher={finisher} k={k} call={call}")


def test_finisher_and_last_arriver_calls_alternate(dev):
    """One sampler, calls that alternate between the finisher hand-off (top-k
    rows only) and the last-arriver one (a greedy row, or log-probs, in the
    batch): each call leaves the workspace as the next one needs it (lists
    cleared, row counters at zero).  Exact against the oracle."""
    rows = 16
    s = fg_hip.HipSampler(W.V, rows)
    for call in range(6):
        w = W.config2(rows=rows)
        w["logits"] = np.roll(w["logits"], 7919 * call, axis=1)  # new data each call
        if call % 3 == 1:
            w["configs"][5] = W.cfg(0.0, 1.0, 1)  # a greedy row
        if call % 3 == 2:
            w["logprobs"] = 5
        check(w, run_hip(w, dev, sampler=s), W.oracle_run(w), f"alternating call {call}")


@pytest.mark.parametrize("groups", [32, 128, 1024])
def test_greedy_finisher_alternates_with_last_arriver(dev, monkeypatch, groups):
    """The greedy finisher (batches of greedy rows: one chunk reads the
    others' words until all carry the launch's epoch) on 2, 8 and
    64 chunks per row, alternating on one sampler with calls whose batch
    mixes in a top-k row (the last-arriver hand-off, which reads the greedy
    slots too and clears them).  Non-finite values win and fail their row
    (src/output.c:560-599), ties go to the lower id; exact against the
    oracle."""
    monkeypatch.setenv("FG_HIP_TARGET_GROUPS", str(groups))
    rows = 16
    s = fg_hip.HipSampler(W.V, rows)
    for call in range(6):
        rng = np.random.default_rng(31 * groups + call)
        logits = rng.normal(0, 3, (rows, W.V)).astype(np.float32)
        logits[1, 77_777] = np.nan
        logits[2, 150_000] = np.inf
        logits[3, [5, 140_000]] = 30.0  # a tie across chunks
        logits[4, :] = -1.0  # every value tied: id 0
        counts = np.zeros((rows, W.V), dtype=np.uint32)
        counts[6, rng.integers(0, W.V, 64)] = 1
        configs = [W.cfg(0.0, 1.0, 1, repetition=1.05 if r == 6 else 1.0) for r in range(rows)]
        if call % 2 == 1:
            configs[9] = W.cfg(0.7, 0.9, 5)  # a top-k row: the last-arriver hand-off
        w = dict(logits=logits, counts=counts, configs=configs,
                 uniforms=rng.random(rows).astype(np.float32), logprobs=0)
        check(w, run_hip(w, dev, sampler=s), W.oracle_run(w),
              f"greedy finisher groups={groups} call={call}")


@pytest.mark.parametrize("greedy", [False, True])
def test_finisher_wait_limit_reports_and_next_call_is_exact(dev, greedy):
    """A finisher whose wait passes its limit reports FG_ERR_UNAVAILABLE (7)
    and token 0xffffffff for its row instead of sampling from the lists it
    has (forced from the host: a limit of 0 us gives up at the first look
    unless every list is in).  The rows that finish are exact.  The other
    workgroups never wait, so the launch completes either way; their lists
    land after the finisher gave up, carrying that launch's epoch, and the
    next calls (limit restored, new data) are exact."""
    rows = 64
    s = fg_hip.HipSampler(W.V, rows)
    w = W.config2(rows=rows)
    if greedy:
        w["configs"] = [W.cfg(0.0, 1.0, 1, presence=1.5, repetition=1.05)] * rows
    s.set_wait_limit(0)
    got = run_hip(w, dev, sampler=s)
    ref = W.oracle_run(w)
    gave_up = got["status"] == 7
    assert gave_up.any(), "a 0 us limit should give up on some row"
    assert (got["token"][gave_up] == 0xFFFFFFFF).all()
    done = ~gave_up
    assert np.array_equal(got["status"][done], ref["status"][done])
    ok = (got["token"][done] == ref["token"][done]) | (ref["margin"][done] < BOUNDARY)
    assert ok.all(), "rows that finished under the limit differ from the oracle"
    s.set_wait_limit(100000)
    for call in range(2):
        w2 = dict(w)
        w2["logits"] = np.roll(w["logits"], 104_729 * (call + 1), axis=1)
        check(w2, run_hip(w2, dev, sampler=s), W.oracle_run(w2), f"after the limit, call {call}")


def test_finisher_epoch_wrap(dev, monkeypatch):
    """The hand-off epoch runs 1..8191 and the workspace is cleared when it
    wraps: 8,200 calls of a two-row batch on one sampler (eight chunks per
    row, the finisher hand-off), the inputs changed before the first, the
    wrapping and the last calls, each of those checked against the
    oracle."""
    import torch
    monkeypatch.setenv("FG_HIP_TARGET_GROUPS", "16")
    rows, vocab = 2, 8192
    s = fg_hip.HipSampler(vocab, rows)
    s.set_configs([fg_hip.make_config(0.9, 0.9, 16, 0.0, 0.0, 1.0)] * rows)
    tok = torch.empty(rows, dtype=torch.int32, device=dev)
    st = torch.empty(rows, dtype=torch.int32, device=dev)
    checks = {0, 8189, 8190, 8191, 8192, 8199}
    for call in range(8200):
        if call in checks:
            rng = np.random.default_rng(call)
            w = dict(logits=rng.normal(0, 2, (rows, vocab)).astype(np.float32),
                     counts=np.zeros((rows, vocab), dtype=np.uint32),
                     configs=[W.cfg(0.9, 0.9, 16)] * rows,
                     uniforms=rng.random(rows).astype(np.float32), logprobs=0)
            x, u = to_dev(w["logits"], dev), to_dev(w["uniforms"], dev)
        s.sample(x, u, tok, row_status=st)
        if call in checks:
            torch.cuda.synchronize()
            got = dict(token=tok.cpu().numpy().view(np.uint32), status=st.cpu().numpy())
            ref = W.oracle_run(w)
            assert np.array_equal(got["status"], ref["status"]), f"call {call}"
            ok = (got["token"] == ref["token"]) | (ref["margin"] < BOUNDARY)
            assert ok.all(), f"call {call}: {got['token']} vs {ref['token']}"


@pytest.mark.parametrize("nucleus", [False, True])
def test_graph_replays_match_eager(dev, nucleus):
    """One sample call captured in a HIP graph (the launch allocates and
    clears nothing: the row counters reset themselves) and replayed three
    times, with eager launches on the same sampler and synchronizations in
    between; every replay's tokens, logits and statuses equal the eager
    call's, which match the oracle."""
    import torch
    rows = 16
    w = W.config3(rows=rows) if nucleus else W.config2(rows=rows)
    flags = fg_hip.ALLOW_FULL_VOCAB if nucleus else 0
    s = fg_hip.HipSampler(W.V, rows)
    eager = run_hip(w, dev, flags=flags, sampler=s)
    check(w, eager, W.oracle_run(w), "eager", NUC_BOUNDARY if nucleus else BOUNDARY)
    d_logits = to_dev(w["logits"], dev)
    d_counts = to_dev(w["counts"], dev)
    d_u = to_dev(w["uniforms"], dev)
    tok = torch.full((rows,), -1, dtype=torch.int32, device=dev)
    tl = torch.zeros(rows, dtype=torch.float32, device=dev)
    st = torch.full((rows,), -1, dtype=torch.int32, device=dev)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            s.sample(d_logits, d_u, tok, counts=d_counts, token_logits=tl, row_status=st,
                     stream=side.cuda_stream)
    torch.cuda.synchronize()
    for replay in range(3):
        tok.fill_(-1)
        st.fill_(-1)
        run_hip(w, dev, flags=flags, sampler=s)  # eager work on the same sampler between replays
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(tok.cpu().numpy().view(np.uint32), eager["token"]), replay
        assert np.array_equal(tl.cpu().numpy().view(np.uint32), eager["logit"].view(np.uint32)), replay
        assert np.array_equal(st.cpu().numpy(), eager["status"]), replay


@pytest.mark.parametrize("greedy", [False, True])
def test_graph_replays_over_new_inputs(dev, greedy):
    """One captured sample call replayed four times in a row, new logits,
    counts and uniforms written into the captured buffers before each
    replay: every replay matches the oracle on its own inputs (a replay
    must not take a word the previous replay left)."""
    import torch
    rows = 16
    s = fg_hip.HipSampler(W.V, rows)
    base = W.config2(rows=rows)
    if greedy:
        for c in base["configs"]:
            c["temperature"] = 0.0
    s.set_configs([fg_hip.make_config(c["temperature"], c["top_p"], c["top_k"], c["presence"],
                                      c["frequency"], c["repetition"]) for c in base["configs"]])
    d_logits = to_dev(base["logits"], dev)
    d_counts = to_dev(base["counts"], dev)
    d_u = to_dev(base["uniforms"], dev)
    tok = torch.full((rows,), -1, dtype=torch.int32, device=dev)
    st = torch.full((rows,), -1, dtype=torch.int32, device=dev)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            s.sample(d_logits, d_u, tok, counts=d_counts, row_status=st, stream=side.cuda_stream)
    torch.cuda.synchronize()
    for replay in range(4):
        rng = np.random.default_rng(500 + replay)
        w = dict(base)
        w["logits"] = rng.normal(0, 2, base["logits"].shape).astype(np.float32)
        w["counts"] = rng.integers(0, 3, base["counts"].shape).astype(np.uint32) * \
            (rng.random(base["counts"].shape) < 0.01)
        w["uniforms"] = rng.random(rows).astype(np.float32)
        d_logits.copy_(torch.from_numpy(w["logits"]))
        d_counts.copy_(torch.from_numpy(w["counts"].astype(np.uint32).view(np.int32)))
        d_u.copy_(torch.from_numpy(w["uniforms"]))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ref = W.oracle_run(w)
        got = tok.cpu().numpy().view(np.uint32)
        assert np.array_equal(st.cpu().numpy(), ref["status"]), replay
        ok = (got == ref["token"]) | (ref["margin"] < BOUNDARY)
        assert ok.all(), (replay, got, ref["token"])


def test_prepared_launch_matches_sample(dev):
    """HipSampler.prepare (the batch marshalled once, launched per call)
    gives the oracle's tokens, call after call on the same buffers."""
    import torch
    w = W.config2(rows=8)
    s = fg_hip.HipSampler(W.V, 8)
    s.set_configs([fg_hip.make_config(c["temperature"], c["top_p"], c["top_k"], c["presence"],
                                      c["frequency"], c["repetition"]) for c in w["configs"]])
    d_logits = to_dev(w["logits"], dev)
    d_counts = to_dev(w["counts"], dev)
    d_u = to_dev(w["uniforms"], dev)
    tok = torch.full((8,), -1, dtype=torch.int32, device=dev)
    st = torch.full((8,), -7, dtype=torch.int32, device=dev)
    launch = s.prepare(d_logits, d_u, tok, counts=d_counts, row_status=st)
    ref = W.oracle_run(w)
    for _ in range(3):
        tok.fill_(-1)
        launch()
        torch.cuda.synchronize()
        got = tok.cpu().numpy().view(np.uint32)
        assert np.array_equal(st.cpu().numpy(), ref["status"])
        ok = ref["margin"] >= BOUNDARY
        assert np.array_equal(got[ok], ref["token"][ok])
