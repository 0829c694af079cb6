"""Vocabulary-split greedy output, host side: the finalist order and combine
(src/output.c:484-497), the split layout (src/protocol.c:23-44, 93-105) and
the owner's combine (src/runtime.c:2440-2466), through the C library.

Pins: the layout against vectors from the reference's compiled
src/protocol.c (tests/golden/ref_split_layout.json); the order against the
reference's known answers (tests/test_fg_vk.c:4067-4070) and its two combine
tests restated (tests/test_fg_vk.c:4021-4065, 4105-4154); the combine against
a brute-force argmax over the whole vocabulary."""
import ctypes as C
import json
import math
from pathlib import Path

import numpy as np
import pytest

import fg_hip
import oracle_ffi as O

GOLDEN = json.loads((Path(__file__).parent / "golden" / "ref_split_layout.json").read_text())
NAN, INF = float("nan"), float("inf")
PAD = 0xFFFFFFFF


def better(a, ai, b, bi):
    return bool(fg_hip.lib().fg_output_better(a, ai, b, bi))


def combine(a, ai, b, bi):
    v, i = C.c_float(0), C.c_uint32(0)
    fg_hip.lib().fg_output_combine(a, ai, b, bi, C.byref(v), C.byref(i))
    return v.value, i.value


def test_layout_matches_reference():
    lib = fg_hip.lib()
    for ways, rank, ok, way in GOLDEN["way_for_rank"]:
        w = C.c_uint32(0xDEAD)
        assert bool(lib.fg_output_split_way_for_rank(ways, rank, C.byref(w))) == ok
        if ok:
            assert w.value == way
    for ways, way, rank in GOLDEN["rank"]:
        assert lib.fg_output_split_rank(ways, way) == rank
    for ways, way, first, rows in GOLDEN["span"]:
        assert fg_hip.split_span(ways, way) == (first, rows)


def test_layout_reference_checks():
    """tests/test_fg_vk.c:4075-4103: spans tile the vocabulary in multiples of
    the 16-row cooking tile (FG_Q8_0_COOK_ROWS)."""
    for ways in (2, 4):
        cursor = 0
        for way in range(ways):
            first, rows = fg_hip.split_span(ways, way)
            assert first == cursor and rows > 0 and rows % 16 == 0
            cursor += rows
        assert cursor == 248320
    assert fg_hip.lib().fg_output_split_way_for_rank(4, 7, None) is False


def test_better_reference_known_answers():
    """tests/test_fg_vk.c:4067-4070."""
    assert better(-1.0, 3, 0.0, PAD) and not better(0.0, PAD, -1.0, 3)
    assert better(NAN, 4, 10.0, 2) and not better(10.0, 2, NAN, 4)
    assert better(2.0, 5, 2.0, 6) and not better(2.0, 6, 2.0, 5)


def test_better_matches_oracle_exhaustive():
    vals = [NAN, INF, -INF, 0.0, -0.0, 1.0, -1.0, 2.5]
    ids = [0, 1, 7, PAD]
    for a in vals:
        for ai in ids:
            for b in vals:
                for bi in ids:
                    want = O.output_better(np.float32(a), ai, np.float32(b), bi)
                    assert better(a, ai, b, bi) == want, (a, ai, b, bi)
                    v, i = combine(a, ai, b, bi)
                    wv, wi = (a, ai) if want else (b, bi)
                    assert i == wi and (v == wv or (math.isnan(v) and math.isnan(wv)))


def _sweep(scores):
    best_v, best_i = float(scores[0]), 0
    for i in range(1, scores.size):
        if better(float(scores[i]), i, best_v, best_i):
            best_v, best_i = float(scores[i]), i
    return best_v, best_i


def _trial_scores(count, trial, step, amp):
    return (np.sin(np.arange(1, count + 1, dtype=np.float32) * np.float32(trial + 1) *
                   np.float32(step)) * np.float32(amp)).astype(np.float32)


def _argbest(s, lo, hi):
    ids = np.arange(lo, hi, dtype=np.uint32)
    j = int(np.lexsort(O.reduce_order_key(s[lo:hi], ids))[0])
    return float(s[lo + j]), lo + j


def test_split_combine_reference_two_way():
    """tests/test_fg_vk.c:4021-4065 restated (the slice argmax by the
    comparator's lexsort, checked against a sequential fg_output_better sweep
    on the full row)."""
    count = 8192
    for trial in range(6):
        s = _trial_scores(count, trial, 0.0031, 3.0)
        if trial == 1:
            s[100] = s[5000] = 5.0
        elif trial == 2:
            s[7] = NAN
        elif trial == 3:
            s[4096] = s[900] = INF
        elif trial == 4:
            s[:] = 1.0
        elif trial == 5:
            s[-1] = 12.0
        ref = _sweep(s)
        assert ref[1] == _argbest(s, 0, count)[1]
        for split in (1, 2, 3):
            boundary = (split * (count // 4) + 15) // 16 * 16
            left, right = _argbest(s, 0, boundary), _argbest(s, boundary, count)
            v, i = combine(left[0], left[1], right[0], right[1])
            assert i == ref[1] and (v == ref[0] or (math.isnan(v) and math.isnan(ref[0])))


def test_split_combine_reference_four_way():
    """tests/test_fg_vk.c:4105-4154 restated, all three combine orders."""
    count, way = 10240, 2560
    for trial in range(8):
        s = _trial_scores(count, trial, 0.0027, 2.0)
        if trial == 1:
            s[10] = s[-1] = 5.0
        elif trial == 2:
            s[way * 2 + 7] = NAN
        elif trial == 3:
            s[way] = s[way * 3 + 3] = INF
        elif trial == 4:
            s[:] = 1.0
        elif trial == 5:
            s[0] = NAN
        elif trial == 6:
            s[way - 1] = 4.0
        elif trial == 7:
            s[way] = s[way + 1] = s[way * 2] = 5.0
        ref = _argbest(s, 0, count)
        slices = [_argbest(s, w * way, (w + 1) * way) for w in range(4)]
        for order in ((0, 1, 2, 3), (3, 1, 0, 2), (2, 0, 3, 1)):
            v, i = slices[order[0]]
            for w in order[1:]:
                v, i = combine(slices[w][0], slices[w][1], v, i)
            assert i == ref[1] and (v == ref[0] or (math.isnan(v) and math.isnan(ref[0])))


def _finalists(ways, local, remote):
    rv = np.array([v for v, _, _ in remote], dtype=np.float32)
    ri = np.array([i for _, i, _ in remote], dtype=np.uint32)
    rr = np.array([r for _, _, r in remote], dtype=np.uint8)
    tok, logit, err = C.c_uint32(0), C.c_float(0), fg_hip.FgError()
    st = fg_hip.lib().fg_output_split_combine_finalists(
        ways, local[0], local[1], rv.ctypes.data, ri.ctypes.data, rr.ctypes.data, len(remote),
        C.byref(tok), C.byref(logit), C.byref(err))
    return st, tok.value, logit.value, err.message.decode()


@pytest.mark.parametrize("ways", [2, 4])
def test_combine_finalists_matches_whole_vocab_argmax(ways):
    rng = np.random.default_rng(ways)
    V = 248320
    spans = [fg_hip.split_span(ways, w) for w in range(ways)]
    for trial in range(5):
        s = rng.normal(0, 2, V).astype(np.float32)
        if trial == 1:
            s[rng.integers(0, V, 3)] = 9.0  # ties across slices
        parts = [_argbest(s, f, f + n) for f, n in spans]
        remote = [(parts[w][0], parts[w][1], (4, 0, 1, 2)[w]) for w in range(1, ways)][::-1]
        st, tok, logit, _ = _finalists(ways, parts[0], remote)
        want = _argbest(s, 0, V)
        assert st == 0 and tok == want[1] and logit == want[0]
        ranks = np.array([0] + [r for _, _, r in remote], dtype=np.uint8)
        vals = [parts[0][0]] + [v for v, _, _ in remote]
        ids = [parts[0][1]] + [i for _, i, _ in remote]
        assert O.split_combine_row(vals, ids, ranks, ways, V, spans)[:2] == (0, want[1])


def test_combine_finalists_errors():
    q = 248320 // 4
    st, _, _, msg = _finalists(4, (1.0, 5), [(2.0, q + 1, 3)])  # rank 3 owns no slice
    assert st == 5 and "owns no slice" in msg
    st, _, _, msg = _finalists(4, (1.0, 5), [(2.0, 5, 0)])  # id outside rank 0's span
    assert st == 5 and "outside rank 0" in msg
    st, _, _, msg = _finalists(2, (NAN, 5), [(2.0, 140048, 0)])
    assert st == 5 and "invalid combined" in msg
    st, _, _, _ = _finalists(2, (1.0, PAD), [(-INF, 140048, 0)])
    assert st == 5
    st, tok, logit, _ = _finalists(2, (1.0, PAD), [(-3.0, 140048, 0)])
    assert st == 0 and tok == 140048 and logit == -3.0
    st, tok, _, _ = _finalists(2, (1.0, 3), [])
    assert st == 0 and tok == 3
