"""GPU parity of the sampled LM head (fg_hip_output_slice_run_dense_sampled:
the Q8_0 product fused with penalties, the top-k ladder and the select,
src/output.c:702-756) against the unfused path on the same inputs: the plain
product's logits (fg_hip_dense_q8_0_cooked) sampled by fg_sampler_hip_sample,
which must agree bit for bit (token, logit bits, status), and sampled by the
C oracle on the host, which must agree under the north-star bar (token ids
bit-exact unless the oracle's draw lies within 1e-6 of a boundary, logits
bit-exact where the tokens agree).  Vocabularies of 4,099 (a partial tile,
one merge group), 151,936 (38 groups) and the reference's 248,320 x 2,560
head (61 groups); greedy rows with and without penalties, top-k 1..64."""
import numpy as np
import pytest

import fg_hip
import workloads as W

pytestmark = pytest.mark.gpu


def cooked_random(rng, width, rows):
    blocks = width // 32
    b = rng.integers(0, 256, (rows, blocks, 34), dtype=np.uint8)
    d = rng.uniform(1e-3, 2e-2, (rows, blocks)).astype(np.float16)
    b[:, :, :2] = d.view(np.uint8).reshape(rows, blocks, 2)
    return fg_hip.cook_q8_0(b.reshape(-1), width, rows)


def token_configs(n, rng):
    base = [W.cfg(0.7, 0.8, 20, presence=1.5, repetition=1.05),   # config 2's controls
            W.cfg(0.0, 1.0, 1, repetition=1.1),                    # greedy, penalised
            W.cfg(0.0, 1.0, 1),                                    # greedy, plain
            W.cfg(1.0, 0.95, 64, presence=1.0, frequency=0.2, repetition=1.05),
            W.cfg(0.6, 1.0, 1),
            W.cfg(1.3, 0.5, 50, frequency=0.5)]
    out = [base[i % len(base)] for i in range(n)]
    rng.shuffle(out)
    return out


def native(configs):
    return [fg_hip.make_config(c["temperature"], c["top_p"], c["top_k"], c["presence"],
                               c["frequency"], c["repetition"]) for c in configs]


def run_both(dev, cooked, hidden, width, vocab, configs, counts_np, uniforms_np, scale):
    """The fused call (twice: the second reuses the workspace the first left)
    and the unfused path; returns (fused, unfused, host logits)."""
    import torch
    tokens = hidden.shape[0]
    counts = torch.from_numpy(counts_np.view(np.int32)).to(dev)
    uniforms = torch.from_numpy(uniforms_np).to(dev)
    sl = fg_hip.OutputSlice(vocab, 1, 0, vocab, tokens)
    tok = torch.full((tokens,), -7, dtype=torch.int32, device=dev)
    lg = torch.zeros(tokens, dtype=torch.float32, device=dev)
    st = torch.full((tokens,), -7, dtype=torch.int32, device=dev)
    for _ in range(2):
        sl.run_dense_sampled(cooked, hidden, width, tokens, native(configs), uniforms, tok, lg, st,
                             counts=counts, scale=scale)
    logits = torch.empty((tokens, vocab), dtype=torch.float32, device=dev)
    fg_hip.dense_q8_0_cooked(logits.view(-1), cooked, hidden, width, vocab, tokens, scale)
    s = fg_hip.HipSampler(vocab, tokens)
    s.set_configs(native(configs))
    tok2 = torch.full((tokens,), -7, dtype=torch.int32, device=dev)
    lg2 = torch.zeros(tokens, dtype=torch.float32, device=dev)
    st2 = torch.full((tokens,), -7, dtype=torch.int32, device=dev)
    s.sample(logits, uniforms, tok2, counts=counts, token_logits=lg2, row_status=st2)
    torch.cuda.synchronize()
    got = dict(token=tok.cpu().numpy().view(np.uint32), logit=lg.cpu().numpy(),
               status=st.cpu().numpy())
    unfused = dict(token=tok2.cpu().numpy().view(np.uint32), logit=lg2.cpu().numpy(),
                   status=st2.cpu().numpy())
    assert np.array_equal(got["status"], unfused["status"]), (got, unfused)
    assert np.array_equal(got["token"], unfused["token"]), (got, unfused)
    assert np.array_equal(got["logit"].view(np.uint32), unfused["logit"].view(np.uint32))
    return got, unfused, logits.cpu().numpy()


@pytest.mark.parametrize("vocab,width,tokens,scale", [(4099, 64, 3, 0.5), (151_936, 512, 6, 0.1),
                                                      (248_320, 2560, 4, 0.05)])
def test_sampled_lm_head_matches_unfused(dev, vocab, width, tokens, scale):
    import torch
    rng = np.random.default_rng(vocab + width)
    cooked = torch.from_numpy(cooked_random(rng, width, vocab)).to(dev)
    hidden = torch.from_numpy(rng.normal(0, 1, (tokens, width)).astype(np.float32)).to(dev)
    counts_np = W.O.build_counts(W.O.gen_zipf_ids(tokens, 1024, vocab, 1.1, vocab, 7), vocab)
    uniforms_np = rng.random(tokens).astype(np.float32)
    configs = token_configs(tokens, rng)
    got, _, logits = run_both(dev, cooked, hidden, width, vocab, configs, counts_np, uniforms_np,
                              scale)
    ref = W.O.sample_rows(configs, logits, uniforms_np, counts=counts_np, threads=8)
    assert np.array_equal(got["status"], ref["status"])
    same = got["token"] == ref["token"]
    assert (same | (ref["margin"] < 1e-6)).all(), (got["token"], ref["token"], ref["margin"])
    assert np.array_equal(got["logit"][same].view(np.uint32), ref["logit"][same].view(np.uint32))


@pytest.mark.parametrize("kind", ["zero_input", "nan_input", "inf_scale_row", "tied_rows"])
def test_sampled_lm_head_special_values(dev, kind):
    """Zero logits (either sign), NaN and infinite logits, and ties, for
    greedy rows with and without penalties and sampled rows: the fused
    result equals the unfused one bit for bit (statuses included)."""
    import torch
    rng = np.random.default_rng(11)
    width, vocab = 128, 3000
    blocks = width // 32
    b = rng.integers(0, 256, (vocab, blocks, 34), dtype=np.uint8)
    d = rng.uniform(1e-3, 2e-2, (vocab, blocks)).astype(np.float16)
    b[:, :, :2] = d.view(np.uint8).reshape(vocab, blocks, 2)
    x = rng.normal(0, 1, (6, width)).astype(np.float32)
    if kind == "zero_input":
        x[:] = 0.0
    elif kind == "nan_input":
        x[1, 7] = np.nan
        x[4, 3] = np.nan
    elif kind == "inf_scale_row":
        b[37, 2, :2] = np.array([0x00, 0x7c], dtype=np.uint8)  # scale +inf in row 37
    else:
        b[100:3000:7] = b[50]  # many rows equal to row 50: tied logits
    cooked = torch.from_numpy(fg_hip.cook_q8_0(b.reshape(-1), width, vocab)).to(dev)
    configs = [W.cfg(0.0, 1.0, 1), W.cfg(0.0, 1.0, 1, presence=0.5),
               W.cfg(0.7, 0.8, 20, presence=1.5, repetition=1.05), W.cfg(1.0, 1.0, 64),
               W.cfg(0.5, 0.9, 3, repetition=1.2), W.cfg(0.0, 1.0, 1, repetition=1.1)]
    counts_np = W.O.build_counts(W.O.gen_uniform_ids(6, 200, vocab, 3, 9), vocab)
    uniforms_np = rng.random(6).astype(np.float32)
    hidden = torch.from_numpy(x).to(dev)
    got, _, logits = run_both(dev, cooked, hidden, width, vocab, configs, counts_np, uniforms_np,
                              0.3)
    if kind == "nan_input":
        assert got["status"][1] == 4 and got["status"][4] == 4  # penalised greedy, sampled
    if kind == "zero_input":
        assert got["status"][0] == 0 and got["token"][0] == 0


def test_sampled_lm_head_argument_errors(dev):
    import torch
    sl = fg_hip.OutputSlice(1000, 1, 0, 1000, 2)
    x = torch.zeros(4096, device=dev)
    out = torch.zeros(4, dtype=torch.int32, device=dev)
    bad = native([W.cfg(0.7, 0.8, 65)])
    with pytest.raises(fg_hip.FgStatusError, match="invalid sampler controls"):
        sl.run_dense_sampled(x, x, 64, 1, bad, x, out, x, out)
    split = fg_hip.OutputSlice(1000, 2, 0, 500, 2)
    with pytest.raises(fg_hip.FgStatusError, match="invalid sampled output arguments"):
        split.run_dense_sampled(x, x, 64, 1, native([W.cfg(0.7, 0.8, 20)]), x, out, x, out)
