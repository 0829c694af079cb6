"""fg_sampler_hip_sample_static (the entry point that allocates nothing: its
workspace is the library's file-scope device array) against
fg_sampler_hip_set_configs + fg_sampler_hip_sample on the same inputs: two
calls in a row, the second with fewer rows and other controls, every output
bit-identical, and both equal to the oracle."""
import numpy as np
import pytest

import fg_hip
import workloads as W

pytestmark = pytest.mark.gpu


def _native(configs):
    return [fg_hip.make_config(c["temperature"], c["top_p"], c["top_k"], c["presence"],
                               c["frequency"], c["repetition"]) for c in configs]


def _run(dev, w, flags, static):
    import torch
    rows, vocab = w["logits"].shape
    L = w["logprobs"]
    x = torch.from_numpy(w["logits"]).to(dev)
    c = torch.from_numpy(w["counts"].view(np.int32)).to(dev)
    u = torch.from_numpy(w["uniforms"]).to(dev)
    tok = torch.full((rows,), -1, dtype=torch.int32, device=dev)
    tl = torch.zeros(rows, dtype=torch.float32, device=dev)
    st = torch.full((rows,), -1, dtype=torch.int32, device=dev)
    lpv = torch.zeros((rows, max(L, 1)), dtype=torch.float32, device=dev)
    lpi = torch.zeros((rows, max(L, 1)), dtype=torch.int32, device=dev)
    kw = dict(counts=c, token_logits=tl, row_status=st, logprobs=L,
              logprob_values=lpv if L else None, logprob_ids=lpi if L else None)
    if static:
        fg_hip.sample_static(vocab, _native(w["configs"]), x, u, tok, flags=flags, **kw)
    else:
        s = fg_hip.HipSampler(vocab, rows)
        s.set_configs(_native(w["configs"]), flags=flags)
        s.sample(x, u, tok, **kw)
    torch.cuda.synchronize()
    return dict(token=tok.cpu().numpy(), logit=tl.cpu().numpy().view(np.uint32),
                status=st.cpu().numpy(), lpv=lpv.cpu().numpy().view(np.uint32),
                lpi=lpi.cpu().numpy())


def _same(a, b, name):
    for k in a:
        assert np.array_equal(a[k], b[k]), f"{name}: {k} differs"


def test_static_matches_sampler_two_calls(dev):
    # Call 1: config 2's 64 rows, some greedy and some top-k 64 rows, with
    # log-probs (several workgroups per row, cross-workgroup hand-off).
    w1 = W.config2(rows=64)
    for r in range(0, 64, 7):
        w1["configs"][r] = W.cfg(0.0, 1.0, 1, repetition=1.1)
    for r in range(3, 64, 11):
        w1["configs"][r] = W.cfg(1.1, 0.95, 64, presence=0.3)
    w1["logprobs"] = 8
    # Call 2: fewer rows, whole-row nucleus controls (a second kernel on the
    # same stream), after call 1 left its contents in the array.
    w2 = W.config3(rows=24)
    # Calls 3 and 4: batches that take the finisher hand-offs (top-k 20 rows
    # only; greedy rows only), after the calls above left their contents.
    w3 = W.config2(rows=16)
    w4 = W.config2(rows=8)
    w4["configs"] = [W.cfg(0.0, 1.0, 1, presence=1.5, repetition=1.05)] * 8
    for k, (w, flags) in enumerate([(w1, 0), (w2, fg_hip.ALLOW_FULL_VOCAB), (w3, 0), (w4, 0)]):
        got = _run(dev, w, flags, static=True)
        want = _run(dev, w, flags, static=False)
        _same(got, want, f"call {k + 1}")
        ref = W.oracle_run(w)
        ok = (got["token"].view(np.uint32) == ref["token"]) | (ref["margin"] < 1e-11)
        assert ok.all() and np.array_equal(got["status"], ref["status"]), f"call {k + 1} vs oracle"


def test_static_rejects_rows_beyond_the_array(dev):
    import torch
    rows = fg_hip.STATIC_MAX_ROWS + 1
    x = torch.zeros((rows, 64), device=dev)
    u = torch.zeros(rows, device=dev)
    tok = torch.zeros(rows, dtype=torch.int32, device=dev)
    cfg = _native([W.cfg(0.0)] * rows)
    with pytest.raises(fg_hip.FgStatusError, match="static sampler workspace"):
        fg_hip.sample_static(64, cfg, x, u, tok)
