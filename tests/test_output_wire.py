"""Output-owner wire messages (include/fg_output_wire.h) against the
reference's compiled codecs: tests/golden/ref_output_wire_vectors.json holds
the encodings and decodings of src/protocol.c:1160-1166, 1275-1279 for valid
messages, every check failing once and byte-wise mutations; both statuses and
bytes / decoded fields must match exactly.  Also the reference's own round
trips (tests/test_core.c:375, tests/test_fabric.c:165-185) and the batch
helpers."""
import ctypes as C
import json
import math
import struct
from pathlib import Path

import pytest

import fg_hip

GOLD = json.loads((Path(__file__).parent / "golden" / "ref_output_wire_vectors.json").read_text())
FIELDS = ("temperature", "top_p", "top_k", "presence_penalty", "frequency_penalty",
          "repetition_penalty", "min_p")


def bits(x):
    return struct.unpack("<I", struct.pack("<f", x))[0]


def from_bits(b):
    return struct.unpack("<f", struct.pack("<I", b))[0]


def make_config(d):
    c = fg_hip.OutputConfig(d["source_rank"], d["destination_rank"], d["flags"], d["session_slot"],
                            d["token_index"])
    for k in FIELDS:
        v = d["sampler"][k]
        setattr(c.sampler, k, v if k == "top_k" else from_bits(v))
    c.uniform = from_bits(d["uniform"])
    return c


def config_dict(c):
    return {"source_rank": c.source_rank, "destination_rank": c.destination_rank,
            "flags": c.flags, "session_slot": c.session_slot, "token_index": c.token_index,
            "sampler": {k: (getattr(c.sampler, k) if k == "top_k" else bits(getattr(c.sampler, k)))
                        for k in FIELDS},
            "uniform": bits(c.uniform)}


def result_dict(r):
    return {"source_rank": r.source_rank, "destination_rank": r.destination_rank,
            "token_index": r.token_index, "token": r.token, "logit": bits(r.logit)}


def test_config_encode_matches_reference():
    lib = fg_hip.lib()
    for v in GOLD["config_encode"]:
        buf = (C.c_uint8 * 40)(*([0xAB] * 40))
        err = fg_hip.FgError()
        st = lib.fg_output_config_encode(buf, C.byref(make_config(v["config"])), C.byref(err))
        assert st == v["status"], v
        if st == 0:
            assert bytes(buf).hex() == v["wire"], v


def test_config_decode_matches_reference():
    lib = fg_hip.lib()
    for v in GOLD["config_decode"]:
        pl = bytes.fromhex(v["payload"])
        buf = (C.c_uint8 * len(pl)).from_buffer_copy(pl)
        c, err = fg_hip.OutputConfig(), fg_hip.FgError()
        st = lib.fg_output_config_decode(C.byref(c), buf, v["bytes"], C.byref(err))
        assert st == v["status"], v
        if st == 0:
            assert config_dict(c) == v["config"], v


def test_result_codec_matches_reference():
    lib = fg_hip.lib()
    for v in GOLD["result_encode"]:
        d = v["result"]
        r = fg_hip.OutputResult(d["source_rank"], d["destination_rank"], d["token_index"],
                                d["token"], from_bits(d["logit"]))
        buf = (C.c_uint8 * 16)(*([0xAB] * 16))
        err = fg_hip.FgError()
        st = lib.fg_output_result_encode(buf, C.byref(r), C.byref(err))
        assert st == v["status"], v
        if st == 0:
            assert bytes(buf).hex() == v["wire"], v
    for v in GOLD["result_decode"]:
        pl = bytes.fromhex(v["payload"])
        buf = (C.c_uint8 * len(pl)).from_buffer_copy(pl)
        r, err = fg_hip.OutputResult(), fg_hip.FgError()
        st = lib.fg_output_result_decode(C.byref(r), buf, v["bytes"], C.byref(err))
        assert st == v["status"], v
        if st == 0:
            assert result_dict(r) == v["result"], v


def test_reference_round_trips():
    """tests/test_core.c:375 (result) and tests/test_fabric.c:165-185 (config)."""
    lib = fg_hip.lib()
    err = fg_hip.FgError()
    r = fg_hip.OutputResult(4, 0, 91, 42, 12.5)
    wire = (C.c_uint8 * 16)()
    assert lib.fg_output_result_encode(wire, C.byref(r), C.byref(err)) == 0
    back = fg_hip.OutputResult()
    assert lib.fg_output_result_decode(C.byref(back), wire, 16, C.byref(err)) == 0
    assert (back.source_rank, back.destination_rank, back.token_index, back.token, back.logit) == \
        (4, 0, 91, 42, 12.5)
    wire[8] = 0xFF  # token >= the vocabulary
    assert lib.fg_output_result_decode(C.byref(back), wire, 16, C.byref(err)) == 4
    c = fg_hip.OutputConfig(0, 4, 0, 0, 17)
    c.uniform = 0.25
    cw = (C.c_uint8 * 40)()
    for flags in (0, 1, 3):
        c.flags = flags
        assert lib.fg_output_config_encode(cw, C.byref(c), C.byref(err)) == 0
        d = fg_hip.OutputConfig()
        assert lib.fg_output_config_decode(C.byref(d), cw, 40, C.byref(err)) == 0
        assert (d.source_rank, d.destination_rank, d.token_index, d.uniform, d.flags) == \
            (0, 4, 17, 0.25, flags)
    for i, v in ((2, 2), (2, 0x80)):
        bad = (C.c_uint8 * 40).from_buffer_copy(bytes(cw))
        bad[i] = v
        assert lib.fg_output_config_decode(C.byref(fg_hip.OutputConfig()), bad, 40, C.byref(err)) != 0
    c.destination_rank = 5
    assert lib.fg_output_config_encode(cw, C.byref(c), C.byref(err)) != 0


def test_batch_helpers():
    lib = fg_hip.lib()
    err = fg_hip.FgError()
    rows = 3
    cfgs = (fg_hip.OutputConfig * rows)()
    cfgs[0] = fg_hip.OutputConfig(0, 4, 0, 0, 5)
    cfgs[0].uniform = 0.5                                    # all controls 0: greedy
    cfgs[1] = fg_hip.OutputConfig(1, 4, 0, 1, 6)
    cfgs[1].sampler = fg_hip.make_config(0.7, 0.8, 20, 1.5, 0.0, 1.05)
    cfgs[1].uniform = 0.25
    cfgs[2] = fg_hip.OutputConfig(2, 4, 0, 0, 7)
    cfgs[2].sampler = fg_hip.make_config(0.0, 1.0, 1, 0.0, 0.0, 1.1)
    samplers = (fg_hip.SamplerConfig * rows)()
    uniforms = (C.c_float * rows)()
    assert lib.fg_output_configs_batch(cfgs, rows, samplers, uniforms, C.byref(err)) == 0
    greedy = fg_hip.SamplerConfig()
    lib.fg_sampler_config_greedy(C.byref(greedy))
    assert bytes(samplers[0]) == bytes(greedy)
    assert bytes(samplers[1]) == bytes(cfgs[1].sampler) and bytes(samplers[2]) == bytes(cfgs[2].sampler)
    assert list(uniforms) == [0.5, 0.25, 0.0]
    for s in samplers:
        assert lib.fg_sampler_config_validate(C.byref(s), C.byref(err)) == 0
    tokens = (C.c_uint32 * rows)(10, 248319, 3)
    logits = (C.c_float * rows)(1.5, -2.0, 0.0)
    status = (C.c_int32 * rows)(0, 0, 4)
    out = (C.c_uint8 * (16 * rows))(*([0xAB] * 16 * rows))
    answered = C.c_uint32(99)
    assert lib.fg_output_results_encode_batch(out, cfgs, tokens, logits, status, rows,
                                              C.byref(answered), C.byref(err)) == 0
    assert answered.value == 2
    for r in range(2):
        back = fg_hip.OutputResult()
        chunk = (C.c_uint8 * 16).from_buffer_copy(bytes(out)[16 * r:16 * r + 16])
        assert lib.fg_output_result_decode(C.byref(back), chunk, 16, C.byref(err)) == 0
        assert (back.source_rank, back.destination_rank, back.token_index, back.token) == \
            (4, cfgs[r].source_rank, cfgs[r].token_index, tokens[r])
    assert bytes(out)[32:48] == bytes(16)
    tokens[0] = 248320  # out of the vocabulary: the encoder's check fails
    assert lib.fg_output_results_encode_batch(out, cfgs, tokens, logits, None, rows,
                                              C.byref(answered), C.byref(err)) == 4
    assert lib.fg_output_configs_batch(None, rows, samplers, uniforms, C.byref(err)) == 2
