"""GPU parity of the vocabulary-split greedy output: per-slice finalists
(fg_hip_output_slice_reduce) against the oracle's restatement of
src/output.c:320-344, the device combine (fg_hip_output_split_combine)
against src/runtime.c:2440-2466 restated, and the two together against the
whole-vocabulary argmax."""
import numpy as np
import pytest

import fg_hip
import oracle_ffi as O

pytestmark = pytest.mark.gpu

Q38 = 248320


def _rows(rng, rows, n, specials=True):
    x = (np.round(rng.normal(0, 3, (rows, n)) * 8) / 8).astype(np.float32)  # many ties
    if specials:
        for r in range(rows):
            kind = r % 6
            if kind == 1:
                x[r, rng.integers(0, n, 2)] = np.nan
            elif kind == 2:
                x[r, rng.integers(0, n, 2)] = np.inf
            elif kind == 3:
                x[r, rng.integers(0, n)] = -np.inf
                x[r, rng.integers(0, n, 3)] = 40.0  # tie at the maximum
            elif kind == 4:
                x[r] = -0.0
                x[r, rng.integers(0, n, 5)] = 0.0
            elif kind == 5:
                x[r, -1] = 50.0  # winner in the last, partial chunk
    return x


def _slice_reduce(dev, sl, x, stride=None, batch=None):
    import torch
    rows = batch if batch is not None else x.shape[0]
    t = torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    if stride is not None:
        padded = torch.full((x.shape[0], stride), 7.0, device=dev)
        padded[:, :x.shape[1]] = t
        t = padded
    vals = torch.empty(rows, dtype=torch.float32, device=dev)
    ids = torch.empty(rows, dtype=torch.int32, device=dev)
    st = torch.empty(rows, dtype=torch.int32, device=dev)
    sl.reduce(t, vals, ids, st, batch_rows=rows)
    torch.cuda.synchronize()
    return vals.cpu().numpy(), ids.cpu().numpy().view(np.uint32), st.cpu().numpy()


def _check(got, want):
    gv, gi, gs = got
    wv, wi, ws = want
    assert np.array_equal(gi, wi)
    assert np.array_equal(gv.view(np.uint32), wv.view(np.uint32))
    assert np.array_equal(gs, ws)


@pytest.mark.parametrize("ways,way", [(2, 0), (2, 1), (4, 0), (4, 3)])
def test_slice_finalists_reference_spans(dev, ways, way):
    first, n = fg_hip.split_span(ways, way)
    rng = np.random.default_rng(ways * 10 + way)
    x = _rows(rng, 24, n)
    sl = fg_hip.OutputSlice(Q38, ways, first, n, 64)
    assert sl.ways() == ways
    _check(_slice_reduce(dev, sl, x), O.slice_finalists(x, first))
    # Second call, fewer rows: the workspace came back to zero.
    y = _rows(rng, 5, n)
    _check(_slice_reduce(dev, sl, y), O.slice_finalists(y, first))


@pytest.mark.parametrize("n,first,stride", [(1, 0, None), (3, 17, None), (8191, 5, None),
                                            (8192, 0, None), (8193, 100, None),
                                            (37_984, 113_952, 38_000), (1001, 9, 1003)])
def test_slice_finalists_shapes(dev, n, first, stride):
    """Scalar path (unaligned stride or odd slice) and vector path, chunk edges."""
    rng = np.random.default_rng(n)
    x = _rows(rng, 12, n)
    sl = fg_hip.OutputSlice(151_936, 4, first, n, 12)
    _check(_slice_reduce(dev, sl, x, stride=stride), O.slice_finalists(x, first))


def test_slice_arguments(dev):
    with pytest.raises(fg_hip.FgStatusError) as e:
        fg_hip.OutputSlice(Q38, 3, 0, 10, 4)
    assert e.value.code == 2 and "invalid output slice arguments" in e.value.message
    with pytest.raises(fg_hip.FgStatusError):
        fg_hip.OutputSlice(Q38, 2, Q38 - 5, 6, 4)
    with pytest.raises(fg_hip.FgStatusError):
        fg_hip.OutputSlice(Q38, 2, 0, 10, 0)
    import torch
    sl = fg_hip.OutputSlice(Q38, 2, 0, 100, 4)
    x = torch.zeros(5, 100, device=dev)
    v = torch.empty(5, device=dev)
    with pytest.raises(fg_hip.FgStatusError):  # more rows than max_batch_rows
        sl.reduce(x, v, v, v, batch_rows=5)
    with pytest.raises(fg_hip.FgStatusError):  # stride below the slice
        sl.reduce(x, v, v, v, batch_rows=2, stride=50)


def _combine(dev, vals, ids, ranks, ways, vocab, spans):
    import torch
    rows = vals.shape[0]
    tv = torch.from_numpy(np.ascontiguousarray(vals, dtype=np.float32)).to(dev)
    ti = torch.from_numpy(np.ascontiguousarray(ids, dtype=np.uint32).view(np.int32)).to(dev)
    tr = torch.from_numpy(np.ascontiguousarray(ranks, dtype=np.uint8)).to(dev)
    tok = torch.empty(rows, dtype=torch.int32, device=dev)
    lg = torch.empty(rows, dtype=torch.float32, device=dev)
    st = torch.empty(rows, dtype=torch.int32, device=dev)
    fg_hip.split_combine(tok, lg, st, tv, ti, tr, rows, ways, vocab, spans)
    torch.cuda.synchronize()
    return tok.cpu().numpy().view(np.uint32), lg.cpu().numpy(), st.cpu().numpy()


@pytest.mark.parametrize("ways", [2, 4])
def test_split_end_to_end_matches_whole_vocab_argmax(dev, ways):
    """Slices reduced on the device, finalists combined on the device: the
    token and logit of the greedy argmax over the whole row."""
    import torch
    rng = np.random.default_rng(40 + ways)
    rows = 32
    x = _rows(rng, rows, Q38)
    spans = [fg_hip.split_span(ways, w) for w in range(ways)]
    vals = np.empty((rows, ways), dtype=np.float32)
    ids = np.empty((rows, ways), dtype=np.uint32)
    status = np.empty((rows, ways), dtype=np.int32)
    tx = torch.from_numpy(x).to(dev)
    for w, (first, n) in enumerate(spans):
        sl = fg_hip.OutputSlice(Q38, ways, first, n, rows)
        view = tx[:, first:first + n]
        v = torch.empty(rows, device=dev)
        i = torch.empty(rows, dtype=torch.int32, device=dev)
        s = torch.empty(rows, dtype=torch.int32, device=dev)
        sl.reduce(view, v, i, s, stride=Q38)
        torch.cuda.synchronize()
        vals[:, w], ids[:, w], status[:, w] = v.cpu().numpy(), u32(i), s.cpu().numpy()
    ranks = np.tile(np.array([0] + [(4, 0, 1, 2)[w] for w in range(1, ways)], np.uint8), (rows, 1))
    tok, lg, st = _combine(dev, vals, ids, ranks, ways, Q38, spans)
    wv, wi, ws = O.slice_finalists(x, 0)
    assert np.array_equal(tok[ws == 0], wi[ws == 0])
    assert np.array_equal(lg[ws == 0].view(np.uint32), wv[ws == 0].view(np.uint32))
    assert np.array_equal(st, ws)  # non-finite whole-row winners fail the combine
    assert np.all(tok[ws != 0] == 0xFFFFFFFF)


def u32(t):
    return t.cpu().numpy().view(np.uint32)


def test_split_combine_matches_oracle_with_bad_partials(dev):
    rng = np.random.default_rng(7)
    ways, vocab, rows = 4, 151_936, 500
    q = vocab // 4
    spans = [(w * q, q) for w in range(4)]
    vals = rng.normal(0, 1, (rows, ways)).astype(np.float32)
    ids = np.empty((rows, ways), dtype=np.uint32)
    ranks = np.zeros((rows, ways), dtype=np.uint8)
    for r in range(rows):
        order = rng.permutation(3) + 1  # remote ways in any order
        ids[r, 0] = rng.integers(0, q)
        for j, w in enumerate(order, start=1):
            ranks[r, j] = (4, 0, 1, 2)[w]
            ids[r, j] = w * q + rng.integers(0, q)
        kind = r % 10
        if kind == 1:
            ranks[r, 2] = 3  # owns no slice
        elif kind == 2:
            ids[r, 1] = ids[r, 0]  # outside its rank's span
        elif kind == 3:
            vals[r, 3] = np.nan  # non-finite winner
        elif kind == 4:
            vals[r, :] = 1.5  # ties: lowest id
        elif kind == 5:
            vals[r, 0] = np.inf
        elif kind == 6:
            ids[r, 0] = 0xFFFFFFFF  # owner padding
        elif kind == 7:
            ids[r, 3] = vocab + 4  # beyond the vocabulary
    tok, lg, st = _combine(dev, vals, ids, ranks, ways, vocab, spans)
    for r in range(rows):
        ws, wt, wv = O.split_combine_row(vals[r], ids[r], ranks[r], ways, vocab, spans)
        assert st[r] == ws and tok[r] == wt, r
        if ws == 0:
            assert lg[r] == np.float32(wv)


def test_split_combine_arguments(dev):
    import torch
    z = torch.zeros(8, dtype=torch.int32, device=dev)
    with pytest.raises(fg_hip.FgStatusError):  # spans do not tile the vocabulary
        fg_hip.split_combine(z, None, z, z, z, z, 2, 2, 100, [(0, 50), (50, 49)])
    with pytest.raises(fg_hip.FgStatusError):
        fg_hip.split_combine(z, None, z, z, z, z, 2, 3, 99, [(0, 33), (33, 33), (66, 33)])


def _parts(rng, rows, ways, vocab, spans, bad=True):
    """Finalists the other ranks sent (way i >= 1 at column i), some bad."""
    vals = rng.normal(0, 2, (rows, ways)).astype(np.float32)
    ids = np.zeros((rows, ways), dtype=np.uint32)
    ranks = np.zeros((rows, ways), dtype=np.uint8)
    for r in range(rows):
        order = rng.permutation(ways - 1) + 1
        for j, w in enumerate(order, start=1):
            ranks[r, j] = (4, 0, 1, 2)[w]
            first, n = spans[w]
            ids[r, j] = first + rng.integers(0, n)
        if bad:
            kind = r % 8
            if kind == 1:
                ranks[r, 1] = 3  # owns no slice
            elif kind == 2:
                vals[r, 1] = 60.0  # beats the owner's slice
            elif kind == 3:
                vals[r, ways - 1] = np.nan
            elif kind == 4:
                ids[r, 1] = vocab + 2
    return vals, ids, ranks


def _step(dev, sl, x, vals, ids, ranks, spans, stride=None):
    import torch
    rows = x.shape[0]
    tx = torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    tv = torch.from_numpy(vals).to(dev)
    ti = torch.from_numpy(ids.view(np.int32)).to(dev)
    tr = torch.from_numpy(ranks).to(dev)
    tok = torch.empty(rows, dtype=torch.int32, device=dev)
    lg = torch.empty(rows, dtype=torch.float32, device=dev)
    st = torch.empty(rows, dtype=torch.int32, device=dev)
    sl.reduce_combine(tx, tv, ti, tr, spans, tok, lg, st)
    torch.cuda.synchronize()
    return u32(tok), lg.cpu().numpy(), st.cpu().numpy()


def _step_two_launches(dev, sl, x, vals, ids, ranks, ways, vocab, spans):
    own_v, own_i, _ = _slice_reduce(dev, sl, x)
    v, i = vals.copy(), ids.copy()
    v[:, 0], i[:, 0] = own_v, own_i
    return _combine(dev, v, i, ranks, ways, vocab, spans)


@pytest.mark.parametrize("ways,rows", [(4, 64), (2, 64), (4, 5)])
def test_slice_step_matches_reduce_then_combine(dev, ways, rows):
    """fg_hip_output_slice_reduce_combine (one launch, tagged hand-off to
    the row's last chunk, which combines) against the two entry points it
    fuses, and against the oracle's combine of the oracle's finalist; three
    calls on one slice with new inputs each."""
    spans = [fg_hip.split_span(ways, w) for w in range(ways)]
    first, n = spans[0]
    sl = fg_hip.OutputSlice(Q38, ways, first, n, 64)
    for call in range(3):
        rng = np.random.default_rng(ways * 100 + rows + call)
        x = _rows(rng, rows, n)
        vals, ids, ranks = _parts(rng, rows, ways, Q38, spans)
        got = _step(dev, sl, x, vals, ids, ranks, spans)
        want = _step_two_launches(dev, sl, x, vals, ids, ranks, ways, Q38, spans)
        assert np.array_equal(got[0], want[0]) and np.array_equal(got[2], want[2])
        ok = want[2] == 0
        assert np.array_equal(got[1][ok].view(np.uint32), want[1][ok].view(np.uint32))
        ov, oi, _ = O.slice_finalists(x, first)
        for r in range(rows):
            v, i = vals[r].copy(), ids[r].copy()
            v[0], i[0] = ov[r], oi[r]
            ws, wt, _ = O.split_combine_row(v, i, ranks[r], ways, Q38, spans)
            assert got[2][r] == ws and got[0][r] == wt, (call, r)


def test_slice_step_graph_replays(dev):
    """A captured step replayed over new inputs written between replays:
    every replay exact (the hand-off's epochs advance on the device)."""
    import torch
    ways, rows = 4, 64
    spans = [fg_hip.split_span(ways, w) for w in range(ways)]
    first, n = spans[0]
    sl = fg_hip.OutputSlice(Q38, ways, first, n, rows)
    tx = torch.zeros(rows, n, device=dev)
    tv = torch.zeros(rows, ways, device=dev)
    ti = torch.zeros(rows, ways, dtype=torch.int32, device=dev)
    tr = torch.zeros(rows, ways, dtype=torch.uint8, device=dev)
    tok = torch.empty(rows, dtype=torch.int32, device=dev)
    lg = torch.empty(rows, dtype=torch.float32, device=dev)
    st = torch.empty(rows, dtype=torch.int32, device=dev)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        sl.reduce_combine(tx, tv, ti, tr, spans, tok, lg, st, stream=s.cuda_stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        sl.reduce_combine(tx, tv, ti, tr, spans, tok, lg, st, stream=s.cuda_stream)
    for rep in range(4):
        rng = np.random.default_rng(900 + rep)
        x = _rows(rng, rows, n)
        vals, ids, ranks = _parts(rng, rows, ways, Q38, spans)
        tx.copy_(torch.from_numpy(x))
        tv.copy_(torch.from_numpy(vals))
        ti.copy_(torch.from_numpy(ids.view(np.int32)))
        tr.copy_(torch.from_numpy(ranks))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        ov, oi, _ = O.slice_finalists(x, first)
        got_t, got_s = u32(tok), st.cpu().numpy()
        for r in range(rows):
            v, i = vals[r].copy(), ids[r].copy()
            v[0], i[0] = ov[r], oi[r]
            ws, wt, _ = O.split_combine_row(v, i, ranks[r], ways, Q38, spans)
            assert got_s[r] == ws and got_t[r] == wt, (rep, r)


def test_slice_step_batches_switch_chunk_size(dev):
    """Batches of 64, 200 and 400 rows on one slice take grids of 2,048-,
    4,096- and 8,192-logit chunks (the smallest resident at once); calls that
    switch between them stay exact against the oracle (a row's hand-off words
    sit at a fixed stride, so no layout reads another row's words)."""
    ways = 4
    spans = [fg_hip.split_span(ways, w) for w in range(ways)]
    first, n = spans[0]
    sl = fg_hip.OutputSlice(Q38, ways, first, n, 400)
    for call, rows in enumerate((64, 200, 400, 64, 200, 64)):
        rng = np.random.default_rng(700 + call)
        x = _rows(rng, rows, n)
        vals, ids, ranks = _parts(rng, rows, ways, Q38, spans)
        tok, _, st = _step(dev, sl, x, vals, ids, ranks, spans)
        ov, oi, _ = O.slice_finalists(x, first)
        for r in range(rows):
            v, i = vals[r].copy(), ids[r].copy()
            v[0], i[0] = ov[r], oi[r]
            ws, wt, _ = O.split_combine_row(v, i, ranks[r], ways, Q38, spans)
            assert st[r] == ws and tok[r] == wt, (call, rows, r)


def test_slice_step_layout_words_survive_epoch_wrap(dev):
    """A 64-row call (2,048-logit chunks, 19 words a row) leaves large bests
    in words 10-17; 8,190 calls of 200 rows (4,096-logit chunks, 10 words)
    then bring rows 0-63's epoch round to the first call's tag.  The next
    64-row call, on smaller logits, must not take those words: each chunk
    layout has its own words and epochs."""
    import torch
    ways = 4
    spans = [fg_hip.split_span(ways, w) for w in range(ways)]
    first, n = spans[0]
    sl = fg_hip.OutputSlice(Q38, ways, first, n, 200)
    rng = np.random.default_rng(808)
    xc = _rows(rng, 64, n, specials=False)
    vals, ids, ranks = _parts(rng, 64, ways, Q38, spans, bad=False)
    _step(dev, sl, xc + np.float32(100.0), vals, ids, ranks, spans)  # tags epoch 1
    rows = 200
    xb = _rows(rng, rows, n, specials=False)
    vb, ib, rb = _parts(rng, rows, ways, Q38, spans, bad=False)
    tx = torch.from_numpy(xb).to(dev)
    tv, ti, tr = (torch.from_numpy(vb).to(dev), torch.from_numpy(ib.view(np.int32)).to(dev),
                  torch.from_numpy(rb).to(dev))
    tok = torch.empty(rows, dtype=torch.int32, device=dev)
    lg = torch.empty(rows, dtype=torch.float32, device=dev)
    st = torch.empty(rows, dtype=torch.int32, device=dev)
    for _ in range(8190):
        sl.reduce_combine(tx, tv, ti, tr, spans, tok, lg, st)
    torch.cuda.synchronize()
    assert int(st.abs().sum()) == 0
    got_t, _, got_s = _step(dev, sl, xc, vals, ids, ranks, spans)
    ov, oi, _ = O.slice_finalists(xc, first)
    for r in range(64):
        v, i = vals[r].copy(), ids[r].copy()
        v[0], i[0] = ov[r], oi[r]
        ws, wt, _ = O.split_combine_row(v, i, ranks[r], ways, Q38, spans)
        assert got_s[r] == ws and got_t[r] == wt, r


def test_slice_wait_limit_reports_and_next_call_is_exact(dev):
    """A wait limit of 0: the row's last chunk gives up on any word not yet there (status
    FG_ERR_UNAVAILABLE, token 0xffffffff) or finishes exactly; the next call,
    with the limit back, is exact."""
    ways, rows = 4, 64
    spans = [fg_hip.split_span(ways, w) for w in range(ways)]
    first, n = spans[0]
    sl = fg_hip.OutputSlice(Q38, ways, first, n, rows)
    rng = np.random.default_rng(31)
    x = _rows(rng, rows, n)
    vals, ids, ranks = _parts(rng, rows, ways, Q38, spans, bad=False)
    want = _step_two_launches(dev, sl, x, vals, ids, ranks, ways, Q38, spans)
    sl.set_wait_limit(0)
    tok, _, st = _step(dev, sl, x, vals, ids, ranks, spans)
    gave_up = st == 7
    assert np.all(tok[gave_up] == 0xFFFFFFFF)
    assert np.array_equal(tok[~gave_up], want[0][~gave_up])
    sl.set_wait_limit(100_000)
    tok, _, st = _step(dev, sl, x, vals, ids, ranks, spans)
    assert np.array_equal(tok, want[0]) and np.array_equal(st, want[2])


def test_slice_step_one_workgroup_a_row(dev):
    """Steps the tagged hand-off does not take (a batch whose grid is not
    resident at once; a slice whose ids reach 2^18): one workgroup a row,
    against the oracle, for the reduction and the fused step."""
    import torch
    ways, rows = 4, 640  # 5 chunks x 640 rows: more workgroups than fit at once
    spans = [fg_hip.split_span(ways, w) for w in range(ways)]
    first, n = spans[0]
    sl = fg_hip.OutputSlice(Q38, ways, first, n, rows)
    rng = np.random.default_rng(61)
    x = _rows(rng, rows, n)
    vals, ids, ranks = _parts(rng, rows, ways, Q38, spans)
    tok, _, st = _step(dev, sl, x, vals, ids, ranks, spans)
    ov, oi, os_ = O.slice_finalists(x, first)
    for r in range(rows):
        v, i = vals[r].copy(), ids[r].copy()
        v[0], i[0] = ov[r], oi[r]
        ws, wt, _ = O.split_combine_row(v, i, ranks[r], ways, Q38, spans)
        assert st[r] == ws and tok[r] == wt, r
    _check(_slice_reduce(dev, sl, x), (ov, oi, os_))
    big, first2 = 400_000, 200_000  # ids up to 399,998
    for n2 in (199_996, 199_999):  # float4 loads; an odd slice: scalar loads
        sl2 = fg_hip.OutputSlice(big, 2, first2, n2, 8)
        y = _rows(rng, 8, n2)
        _check(_slice_reduce(dev, sl2, y), O.slice_finalists(y, first2))


def test_slice_step_arguments(dev):
    import torch
    spans = [fg_hip.split_span(4, w) for w in range(4)]
    first, n = spans[0]
    sl = fg_hip.OutputSlice(Q38, 4, first, n, 8)
    x = torch.zeros(8, n, device=dev)
    z = torch.zeros(32, dtype=torch.int32, device=dev)
    with pytest.raises(fg_hip.FgStatusError):  # spans do not tile the vocabulary
        sl.reduce_combine(x, z, z, z, spans[:3], z, None, z)
    with pytest.raises(fg_hip.FgStatusError):  # more rows than max_batch_rows
        sl.reduce_combine(x, z, z, z, spans, z, None, z, batch_rows=9)
    with pytest.raises(fg_hip.FgStatusError):
        sl.set_wait_limit(10**9)
    whole = fg_hip.OutputSlice(Q38, 1, 0, Q38, 8)  # one way: nothing to combine
    with pytest.raises(fg_hip.FgStatusError):
        whole.reduce_combine(torch.zeros(8, Q38, device=dev), z, z, z, [(0, Q38)], z, None, z)
