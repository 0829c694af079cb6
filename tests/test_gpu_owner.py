"""The output owner's loop end to end: output configs travel as 40-byte wire
messages (include/fg_output_wire.h, the reference's src/protocol.c:1160-1166
format), are decoded, turned into one batch (fg_output_configs_batch),
sampled in one launch (fg_sampler_hip_sample) and answered as 16-byte
results (fg_output_results_encode_batch).  The decoded answers must carry the
oracle's tokens and logits for the same rows, controls and draws."""
import ctypes as C

import numpy as np
import pytest

import fg_hip
import workloads as W

pytestmark = pytest.mark.gpu


def test_owner_loop_matches_oracle(dev):
    import torch
    lib = fg_hip.lib()
    err = fg_hip.FgError()
    rng = np.random.default_rng(44)
    rows, vocab = 16, 20_000
    logits = rng.normal(0, 3, (rows, vocab)).astype(np.float32)
    counts = np.zeros((rows, vocab), dtype=np.uint32)
    for r in range(rows):
        counts[r, rng.integers(0, vocab, 64)] += 1
    controls = []
    for r in range(rows):
        if r % 4 == 0:
            controls.append(None)                                    # no controls: greedy
        elif r % 4 == 1:
            controls.append((0.7, 0.8, 20, 1.5, 0.0, 1.05))
        elif r % 4 == 2:
            controls.append((1.0, 0.95, 64, 0.5, 0.3, 1.0))
        else:
            controls.append((0.0, 1.0, 1, 0.0, 0.0, 1.1))           # greedy with repetition
    uniforms = rng.random(rows).astype(np.float32)
    wires = []
    for r in range(rows):
        c = fg_hip.OutputConfig(0, 4, 0, r % 2, 1000 + r)
        if controls[r] is not None:
            c.sampler = fg_hip.make_config(*controls[r])
            c.sampler.seed = 0
        c.uniform = float(uniforms[r])
        buf = (C.c_uint8 * 40)()
        assert lib.fg_output_config_encode(buf, C.byref(c), C.byref(err)) == 0, err.message
        wires.append(bytes(buf))
    # The owner's side: decode, batch, sample, answer.
    cfgs = (fg_hip.OutputConfig * rows)()
    for r, w in enumerate(wires):
        buf = (C.c_uint8 * 40).from_buffer_copy(w)
        assert lib.fg_output_config_decode(C.byref(cfgs[r]), buf, 40, C.byref(err)) == 0
    samplers = (fg_hip.SamplerConfig * rows)()
    us = (C.c_float * rows)()
    assert lib.fg_output_configs_batch(cfgs, rows, samplers, us, C.byref(err)) == 0
    s = fg_hip.HipSampler(vocab, rows)
    s.set_configs(list(samplers))
    d_logits = torch.from_numpy(logits).to(dev)
    d_counts = torch.from_numpy(counts.view(np.int32)).to(dev)
    d_u = torch.tensor(list(us), dtype=torch.float32, device=dev)
    tok = torch.empty(rows, dtype=torch.int32, device=dev)
    tl = torch.empty(rows, dtype=torch.float32, device=dev)
    st = torch.empty(rows, dtype=torch.int32, device=dev)
    s.sample(d_logits, d_u, tok, counts=d_counts, token_logits=tl, row_status=st)
    torch.cuda.synchronize()
    tokens = tok.cpu().numpy().view(np.uint32)
    tlog = tl.cpu().numpy()
    status = st.cpu().numpy()
    out = (C.c_uint8 * (16 * rows))()
    answered = C.c_uint32()
    assert lib.fg_output_results_encode_batch(
        out, cfgs, (C.c_uint32 * rows)(*tokens.tolist()), (C.c_float * rows)(*tlog.tolist()),
        (C.c_int32 * rows)(*status.tolist()), rows, C.byref(answered), C.byref(err)) == 0
    assert answered.value == rows
    # The oracle on the same rows (all-zero controls sample as greedy).
    configs = [W.cfg(0.0, 1.0, 1) if c is None else
               W.cfg(c[0], c[1], c[2], presence=c[3], frequency=c[4], repetition=c[5])
               for c in controls]
    ref = W.oracle_run(dict(logits=logits, counts=counts, configs=configs, uniforms=uniforms,
                            logprobs=0))
    for r in range(rows):
        res = fg_hip.OutputResult()
        chunk = (C.c_uint8 * 16).from_buffer_copy(bytes(out)[16 * r:16 * r + 16])
        assert lib.fg_output_result_decode(C.byref(res), chunk, 16, C.byref(err)) == 0
        assert (res.source_rank, res.destination_rank, res.token_index) == (4, 0, 1000 + r)
        assert ref["status"][r] == 0
        if ref["margin"][r] >= 1e-6:
            assert res.token == ref["token"][r], r
            assert np.float32(res.logit).view(np.uint32) == np.float32(ref["logit"][r]).view(np.uint32)
