"""Output-history wire format (include/fg_history.h): the host codec against
the reference's own compiled encoder/decoder (golden vectors from
tests/golden/make_history_golden.py) and the reference test's known answers
(tests/test_core.c:944-975); the oracle's restated decoder against the same
vectors.  The device decoder is tested in tests/test_gpu_units.py."""
import json
import struct
from pathlib import Path

import pytest

import fg_hip
import oracle_ffi as O

GOLDEN = json.loads((Path(__file__).parent / "golden" / "ref_history_vectors.json").read_text())
V = GOLDEN["vocab"]


@pytest.mark.parametrize("case", GOLDEN["encode"], ids=lambda c: f"n{len(c['tokens'])}s{c['slot']}c{c['capacity']}")
def test_encode_matches_reference(case):
    if case["status"] == 0:
        got = fg_hip.history_encode(case["tokens"], case["slot"], capacity=case["capacity"])
        assert got.hex() == case["payload"]
    else:
        with pytest.raises(fg_hip.FgStatusError) as e:
            fg_hip.history_encode(case["tokens"], case["slot"], capacity=case["capacity"])
        assert e.value.code == case["status"]


@pytest.mark.parametrize("case", GOLDEN["decode"], ids=lambda c: f"b{len(c['payload']) // 2}c{c['capacity']}")
def test_decode_matches_reference(case):
    data = bytes.fromhex(case["payload"])
    if case["status"] == 0:
        tokens, slot = fg_hip.history_decode(data, case["capacity"])
        assert tokens == case["tokens"] and slot == case["slot"]
    else:
        with pytest.raises(fg_hip.FgStatusError) as e:
            fg_hip.history_decode(data, case["capacity"])
        assert e.value.code == case["status"]
    st, tokens, slot = O.history_decode(data, case["capacity"], V)
    assert st == case["status"]
    if st == 0:
        assert tokens == case["tokens"] and slot == case["slot"]


def test_reference_known_answers():
    # tests/test_core.c:944-975
    wire = fg_hip.history_encode([7, 7, 42])
    assert len(wire) == fg_hip.HISTORY_HEADER_BYTES + 12
    assert fg_hip.history_decode(wire, 8) == ([7, 7, 42], 0)
    empty = fg_hip.history_encode([])
    assert len(empty) == fg_hip.HISTORY_HEADER_BYTES
    assert fg_hip.history_decode(empty, 0) == ([], 0)
    bad = bytearray(empty)
    bad[4] = 2  # FG_DECODE_BATCH_MAX_SLOTS
    with pytest.raises(fg_hip.FgStatusError) as e:
        fg_hip.history_decode(bytes(bad), 8)
    assert e.value.code == fg_hip.FG_ERR_FORMAT
    bad[4], bad[3] = 0, 1
    with pytest.raises(fg_hip.FgStatusError) as e:
        fg_hip.history_decode(bytes(bad), 8)
    assert e.value.code == fg_hip.FG_ERR_FORMAT
    with pytest.raises(fg_hip.FgStatusError) as e:
        fg_hip.history_decode(empty[:-1], 8)
    assert e.value.code == fg_hip.FG_ERR_ARGUMENT
    tok = bytearray(wire)
    tok[8:12] = b"\xff\xff\xff\xff"
    with pytest.raises(fg_hip.FgStatusError) as e:
        fg_hip.history_decode(bytes(tok), 8)
    assert e.value.code == fg_hip.FG_ERR_FORMAT


def test_vocab_parameter():
    """The _vocab forms check tokens against the given vocabulary."""
    wire = fg_hip.history_encode([151_935, 3], 1, vocab=151_936)
    assert wire == struct.pack(">IB3xII", 2, 1, 151_935, 3)
    assert fg_hip.history_decode(wire, 2, vocab=151_936) == ([151_935, 3], 1)
    with pytest.raises(fg_hip.FgStatusError):
        fg_hip.history_encode([151_936], vocab=151_936)
    with pytest.raises(fg_hip.FgStatusError):
        fg_hip.history_decode(struct.pack(">IB3xI", 1, 0, 151_936), 1, vocab=151_936)
    assert O.history_decode(struct.pack(">IB3xI", 1, 0, 151_936), 1, 151_936)[0] == 4
