"""Pins the CPU oracle (oracle/fg_oracle.c) before it is trusted as the
checker: against the reference's own outputs (golden vectors from its
compiled sources), the known answers of the reference's tests, published
known-answer vectors, closed forms and brute force."""
import json
import math
import struct
from pathlib import Path

import numpy as np
import pytest

import oracle_ffi as O

GOLDEN = json.loads((Path(__file__).parent / "golden" / "ref_sampler_vectors.json").read_text())


def f32(bits):
    return np.array(bits, dtype=np.uint32).view(np.float32)


def fbits(x):
    return struct.unpack("<I", struct.pack("<f", np.float32(x)))[0]


# ---- Philox4x32-10: Random123 known-answer vectors ---------------------------

@pytest.mark.parametrize("ctr,key,want", [
    ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
    ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
    ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
     [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
])
def test_philox_known_answers(ctr, key, want):
    assert O.philox(ctr, key).tolist() == want


# ---- fg_sampler_select (src/sampler.c:80-122) ----------------------------------

def test_select_matches_reference_vectors():
    for c in GOLDEN["select"]:
        s = f32(c["scores_bits"])
        st, tok, logit, cut, margin = O.select(c["t"], c["p"], c["k"], s,
                                               np.array(c["ids"], dtype=np.uint32),
                                               f32([c["u_bits"]])[0])
        assert st == c["status"], c
        if st == 0:
            assert tok == c["token"], c
            assert fbits(logit) == c["logit_bits"], c


def test_select_known_answers_of_reference_test():
    """tests/test_sampler.c:31-46 (scores {5,4,3}, ids {9,3,1})."""
    s = np.array([5, 4, 3], dtype=np.float32)
    ids = np.array([9, 3, 1], dtype=np.uint32)
    assert O.select(1.0, 1.0, 3, s, ids, 0.8)[1] == 3
    assert O.select(0.1, 1.0, 3, s, ids, 0.8)[1] == 9
    assert O.select(0.1, 0.5, 3, s, ids, 0.99)[1] == 9
    assert O.select(0.01, 1.0, 3, s, ids, 0.99)[1] == 9
    assert O.select(1.0, 1.0, 2, s, ids, 0.3)[1] != 1
    assert O.select(0.0, 1.0, 1, np.array([1, 1], np.float32), np.array([8, 2], np.uint32), 0.5)[1] == 2


def brute_select(t, p, k, s, ids, u):
    """Independent restatement with Python floats and math.exp (sequential sums)."""
    c = sorted([(float(v), int(i)) for v, i in zip(s, ids) if math.isfinite(v)],
               key=lambda x: (-x[0], x[1]))
    if not c:
        return 4, None
    if t == 0:
        return 0, c[0][1]
    lim = min(k, len(c)) if k else len(c)
    m = c[0][0]
    tot = sum(math.exp(c[i][0] - m) for i in range(lim))
    cum, cut = 0.0, lim
    for i in range(lim):
        cum += math.exp(c[i][0] - m) / tot
        if cum >= float(np.float32(p)):
            cut = i + 1
            break
    mt = c[0][0] / float(np.float32(t))
    ts = sum(math.exp(c[i][0] / float(np.float32(t)) - mt) for i in range(cut))
    uu = float(np.float32(u))
    if not math.isfinite(uu) or uu < 0:
        uu = 0.0
    if uu >= 1.0:
        uu = float(np.nextafter(np.float32(1), np.float32(0)))
    d = uu * ts
    run = 0.0
    for i in range(cut):
        run += math.exp(c[i][0] / float(np.float32(t)) - mt)
        if d < run:
            return 0, c[i][1]
    return 0, c[cut - 1][1]


def test_select_whole_row_nucleus_matches_brute_force():
    """top_k = 0 (the whole-vocabulary extension) on small rows."""
    rng = np.random.default_rng(3)
    for _ in range(60):
        n = int(rng.integers(1, 400))
        s = (rng.normal(0, rng.choice([0.3, 1, 3]), n)).astype(np.float32)
        ids = np.arange(n, dtype=np.uint32)
        t = float(rng.choice([0.5, 1.0, 2.0]))
        p = float(rng.choice([0.5, 0.9, 0.95, 1.0]))
        u = float(rng.random())
        st, tok, logit, cut, margin = O.select(t, p, 0, s, ids, u)
        bst, btok = brute_select(t, p, 0, s, ids, u)
        assert st == bst
        if margin > 1e-9:
            assert tok == btok


# ---- penalties (src/sampler.c:46-60) ----------------------------------------------

def test_penalties_match_reference_vectors():
    for c in GOLDEN["penalties"]:
        s = f32(c["scores_bits"])
        counts = np.array(c["counts"], dtype=np.uint32)
        out = O.penalties_c(s, counts, c["presence"], c["frequency"], c["repetition"])
        assert out.view(np.uint32).tolist() == c["out_bits"]


def test_penalties_known_answer_of_reference_test():
    """tests/test_sampler.c:48-53: p=1, f=.5, r=2 on [4,-4,3] with counts
    [2,3,0] (ids 1,2,3 into {0,2,3,0}) -> [0, -10.5, 3]."""
    out = O.penalties_c(np.array([4, -4, 3], np.float32), np.array([2, 3, 0], np.uint32), 1.0, 0.5, 2.0)
    assert out.tolist() == [0.0, -10.5, 3.0]


def test_penalties_glsl_rounding_differs_by_one_intermediate_rounding():
    """shaders/fg_apply_penalties.comp:18 rounds (s - f*c) - p, the C API
    s - (f*c + p): the two differ by at most one rounding of the largest
    intermediate (so by <= 1 ulp of the result unless the result cancels)."""
    rng = np.random.default_rng(5)
    s = rng.normal(0, 5, 50_000).astype(np.float32)
    c = rng.integers(0, 50, s.size).astype(np.uint32)
    a = O.penalties_c(s, c, 0.5, 0.3, 1.0).astype(np.float64)
    b = O.penalties_glsl(s, c, 0.5, 0.3, 1.0).astype(np.float64)
    scale = np.maximum(np.maximum(np.abs(s), 0.3 * c + 0.5), np.abs(a)).astype(np.float32)
    assert np.all(np.abs(a - b) <= np.spacing(scale).astype(np.float64))
    same = np.abs(a) >= 0.25 * scale  # no cancellation
    rel = np.abs(a - b)[same] / np.abs(a[same])
    assert rel.max() <= 1e-6


# ---- xorshift64* (src/sampler.c:62-73) ---------------------------------------------

def test_uniform_streams_match_reference_vectors():
    import ctypes as C
    for c in GOLDEN["uniforms"]:
        seed = int(c["seed"])
        st = C.c_uint64(seed if seed else 0x9E3779B97F4A7C15)
        got = [fbits(O.oracle().fgo_xorshift_uniform(C.byref(st))) for _ in range(16)]
        assert got == c["uniform_bits"]


def test_uniform_closed_form():
    import ctypes as C
    x = 42
    st = C.c_uint64(42)
    for _ in range(8):
        x ^= x >> 12
        x ^= (x << 25) & (2**64 - 1)
        x ^= x >> 27
        want = float(np.float32(((x * 2685821657736338717) % 2**64 >> 40) / 16777216.0))
        assert O.oracle().fgo_xorshift_uniform(C.byref(st)) == want


# ---- argmax ladder (shaders/fg_argmax_reduce.comp, src/output.c:484-492) -------------

def ladder_argmax(s):
    v, i = O.argmax_reduce_step(s)
    while v.size > 1:
        v, i = O.argmax_reduce_step(v, i)
    return float(v[0]), int(i[0])


def test_argmax_known_answers_of_reference_test():
    """tests/test_fg_vk.c:1340-1342."""
    s = -np.arange(248_320, dtype=np.float32)
    s[12345] = s[23456] = 100
    assert ladder_argmax(s) == (100.0, 12345)
    s[45678] = np.nan
    v, i = ladder_argmax(s)
    assert i == 45678 and math.isnan(v)


def test_argmax_step_brute_force():
    rng = np.random.default_rng(11)
    for trial in range(5):
        n = int(rng.integers(1, 20_000))
        s = np.round(rng.normal(0, 1, n), 1).astype(np.float32)
        if trial == 3:
            s[rng.integers(0, n, 5)] = -np.inf
        ids = rng.permutation(n).astype(np.uint32)
        v, i = O.argmax_reduce_step(s, ids)
        for g in range(v.size):
            seg = slice(g * 4096, min(n, (g + 1) * 4096))
            ss, ii = s[seg], ids[seg]
            bad = ~np.isfinite(ss)
            if bad.any():
                want = int(ii[bad].min())
            else:
                best = ss.max()
                want = int(ii[ss == best].min())
            assert int(i[g]) == want


# ---- top-k ladder (shaders/fg_topk_select.comp) ---------------------------------------

def test_topk_known_answers_of_reference_test():
    """tests/test_fg_vk.c:1274-1338."""
    s = np.array([1, 9, 7, 9, 3, 8, 2, 7, 6, 5, 4, 0, -1, -2, -3, -4, -5, -6, np.nan], np.float32)
    v, i = O.topk_select_step(s, 4)
    assert sorted(i.tolist()) == [1, 2, 3, 5]
    v, i = O.topk_select_step(s, 1)
    assert i.tolist() == [1]
    short = np.full(19, np.nan, np.float32)
    short[1], short[3] = 9, 8
    v, i = O.topk_select_step(short, 4)
    assert i[0] != O.INVALID_ID and i[1] != O.INVALID_ID and i[2] == O.INVALID_ID
    assert not np.isfinite(v[2])


def key_np(s):
    b = s.view(np.uint32).astype(np.uint64)
    k = np.where(b & 0x80000000, (~b) & 0xFFFFFFFF, b | 0x80000000)
    return np.where(np.isfinite(s), k, 0)


def test_topk_row_equals_full_sort():
    rng = np.random.default_rng(13)
    for trial in range(20):
        n = int(rng.integers(1, 5000))
        s = np.round(rng.normal(0, 2, n) * 4) / 4
        s = s.astype(np.float32)
        s[rng.integers(0, n, n // 50 + 1)] = rng.choice([np.nan, np.inf, -np.inf, 0.0, -0.0])
        k = int(rng.integers(1, 65))
        v, i, have = O.topk_row(s, k)
        keys = key_np(s)
        order = np.lexsort((np.arange(n), -keys.astype(np.float64)))
        order = [j for j in order if keys[j] != 0][:k]
        assert have == len(order)
        assert i[:have].tolist() == order
        assert (i[have:] == O.INVALID_ID).all()


def test_topk_step_sets_equal_tile_sort():
    rng = np.random.default_rng(17)
    s = np.round(rng.normal(0, 2, 5000) * 2) / 2
    s = s.astype(np.float32)
    s[::97] = np.nan
    for k in (1, 7, 20, 64):
        v, i = O.topk_select_step(s, k)
        for t in range((s.size + 1023) // 1024):
            tile = s[t * 1024:(t + 1) * 1024]
            keys = key_np(tile)
            order = np.lexsort((np.arange(tile.size), -keys.astype(np.float64)))
            want = sorted([int(j) + t * 1024 for j in order if keys[j] != 0][:k])
            got = [int(x) for x in i[t * k:(t + 1) * k] if x != O.INVALID_ID]
            assert got == want  # tile order


# ---- whole rows: log-probs closed form ------------------------------------------------

def test_logprobs_closed_form():
    rng = np.random.default_rng(19)
    n = 3000
    logits = rng.normal(0, 4, (3, n)).astype(np.float32)
    logits[1, 5] = np.inf
    cfgs = [dict(temperature=0.6, top_p=0.95, top_k=64), dict(temperature=1.0, top_p=0.9, top_k=8),
            dict(temperature=0.0, top_p=1.0, top_k=1)]
    out = O.sample_rows(cfgs, logits, np.full(3, 0.5, np.float32), logprobs=20)
    for r in range(3):
        t = cfgs[r]["temperature"] or 1.0
        x = logits[r].astype(np.float64)
        fin = np.isfinite(x)
        lse = np.log(np.sum(np.exp(x[fin] / t - (x[fin] / t).max()))) + (x[fin] / t).max()
        kk = max(cfgs[r]["top_k"], 20) if cfgs[r]["temperature"] > 0 else 20
        order = [j for j in np.lexsort((np.arange(n), -np.where(fin, x, -np.inf))) if fin[j]][:kk]
        order = sorted(order, key=lambda j: (-x[j], j))[:20]
        assert out["lp_ids"][r].tolist() == order
        np.testing.assert_allclose(out["lp_values"][r], x[order] / t - lse, atol=1e-5)


def test_greedy_row_status():
    logits = np.array([[1, 2, np.nan, 3], [1, 5, 2, 3], [np.nan] * 4], dtype=np.float32)
    cfgs = [dict(temperature=0.0, top_p=1.0, top_k=1)] * 3
    out = O.sample_rows(cfgs, logits, np.zeros(3, np.float32))
    assert out["status"].tolist() == [5, 0, 5]
    assert out["token"][1] == 1


def test_generators_shapes_and_moments():
    x = O.gen_logits(2, 100_000, 0, 3.0, seed=9, config_id=2)
    assert abs(x.std() - 3.0) < 0.05 and abs(x.mean()) < 0.05
    q = O.gen_logits(1, 50_000, 2, 3.0, seed=9, config_id=4)
    assert np.all(np.abs(q) <= 16) and np.all(q * 4 == np.round(q * 4))
    ids = O.gen_zipf_ids(1, 200_000, 151_936, 1.1, 5, 5)
    counts = np.bincount(ids.ravel(), minlength=151_936)
    top = np.sort(counts)[::-1]
    # Zipf(1.1): rank 1 carries about 1/H share, rank 2 about 2^-1.1 of rank 1.
    assert 0.4 < top[1] / top[0] < 0.55


def test_topk_reduce_order_matches_pairwise_comparator():
    """The oracle's lexsort order against the comparator applied pairwise
    (insertion sort, brute force) on small tiles with NaN, +-Inf, +-0, ties
    and padding ids."""
    import functools
    rng = np.random.default_rng(5)
    for trial in range(40):
        n = int(rng.integers(1, 40))
        s = np.round(rng.normal(0, 2, n) * 2) / 2
        s[rng.random(n) < 0.1] = np.nan
        s[rng.random(n) < 0.05] = np.inf
        s[rng.random(n) < 0.05] = -np.inf
        s[rng.random(n) < 0.1] = -0.0
        s = s.astype(np.float32)
        ids = rng.choice(10_000, n, replace=False).astype(np.uint32)
        ids[rng.random(n) < 0.1] = 0xFFFFFFFF
        cmp = lambda x, y: -1 if O.reduce_before(s[x], ids[x], s[y], ids[y]) else (
            1 if O.reduce_before(s[y], ids[y], s[x], ids[x]) else 0)
        brute = sorted(range(n), key=functools.cmp_to_key(cmp))
        got_s, got_i = O.topk_reduce_step(s, ids)
        want_i = ids[brute][:got_i.size]
        # padding entries tie with each other: compare the non-padding prefix exactly
        real = want_i != 0xFFFFFFFF
        assert np.array_equal(got_i[:real.sum()], want_i[real]), trial
        assert np.array_equal(got_s[:real.sum()].view(np.uint32),
                              s[brute][:got_i.size][real].view(np.uint32))
