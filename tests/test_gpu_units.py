"""GPU parity of the unit entry points that replace the reference's Vulkan
dispatches: penalties, the argmax ladder and the top-k ladder, plus the
history table kernels.  Known answers are the reference's own GPU tests
(tests/test_fg_vk.c:1274-1342)."""
import numpy as np
import pytest

import fg_hip
import oracle_ffi as O
import workloads as W

pytestmark = pytest.mark.gpu


def dev_f32(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def dev_u32(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).to(dev)


def u32(t):
    return t.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("vocab,offset", [(151_936, 0), (248_320, 0), (1001, 0), (4099, 1)])
def test_apply_penalties_matches_c_formula(dev, vocab, offset):
    import torch
    rng = np.random.default_rng(vocab)
    x = rng.normal(0, 3, vocab + offset).astype(np.float32)
    c = np.zeros(vocab + offset, dtype=np.uint32)
    hot = rng.integers(0, vocab + offset, 5000)
    c[hot] = rng.integers(1, 1000, hot.size).astype(np.uint32)
    c[:3] = [0xFFFFFFFF, 7, 1]
    x[:3] = [-0.0, 0.0, np.nan]
    dx = dev_f32(x, dev)
    dc = dev_u32(c, dev)
    fg_hip.apply_penalties(dx[offset:], dc[offset:], 1.5, 0.3, 1.05)
    torch.cuda.synchronize()
    want = O.penalties_c(x[offset:], c[offset:], 1.5, 0.3, 1.05)
    got = dx[offset:].cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_apply_penalties_rejects_bad_arguments(dev):
    x = dev_f32(np.zeros(8), dev)
    c = dev_u32(np.zeros(8), dev)
    for pres, freq, rep in [(np.nan, 0, 1), (0, np.inf, 1), (0, 0, 0.0), (0, 0, -1.0)]:
        with pytest.raises(fg_hip.FgStatusError) as e:
            fg_hip.apply_penalties(x, c, pres, freq, rep)
        assert e.value.code == fg_hip.FG_ERR_ARGUMENT


def ladder_argmax(scores, dev):
    import torch
    n = scores.size
    cur_s = dev_f32(scores, dev)
    cur_i = None
    while n > 1:
        g = (n + 4095) // 4096
        os_ = torch.empty(g, dtype=torch.float32, device=dev)
        oi = torch.empty(g, dtype=torch.int32, device=dev)
        n = fg_hip.argmax_reduce(os_, oi, cur_s, cur_i, n)
        cur_s, cur_i = os_, oi
    torch.cuda.synchronize()
    return float(cur_s.cpu()[0]), int(u32(cur_i)[0]) if cur_i is not None else 0


def test_argmax_known_answers(dev):
    """tests/test_fg_vk.c:1340-1342: s_i = -i, s[12345] = s[23456] = 100 -> 12345;
    then s[45678] = NaN -> 45678 (non-finite ranks first)."""
    n = 248_320
    s = -np.arange(n, dtype=np.float32)
    s[12345] = 100.0
    s[23456] = 100.0
    v, i = ladder_argmax(s, dev)
    assert (i, v) == (12345, 100.0)
    s[45678] = np.nan
    v, i = ladder_argmax(s, dev)
    assert i == 45678 and not np.isfinite(v)


@pytest.mark.parametrize("seed", range(4))
def test_argmax_step_matches_oracle(dev, seed):
    import torch
    rng = np.random.default_rng(seed)
    n = 50_000 + seed * 777
    s = np.round(rng.normal(0, 2, n), 1).astype(np.float32)  # many ties
    ids = rng.permutation(n).astype(np.uint32)
    ids[::97] = 0xFFFFFFFF  # padding entries
    if seed == 1:
        s[rng.integers(0, n, 20)] = np.inf
    if seed == 2:
        s[:] = 0.0
        s[::2] = -0.0
    g = (n + 4095) // 4096
    os_ = torch.empty(g, dtype=torch.float32, device=dev)
    oi = torch.empty(g, dtype=torch.int32, device=dev)
    assert fg_hip.argmax_reduce(os_, oi, dev_f32(s, dev), dev_u32(ids, dev), n) == g
    torch.cuda.synchronize()
    ws, wi = O.argmax_reduce_step(s, ids)
    assert np.array_equal(u32(oi), wi)
    assert np.array_equal(os_.cpu().numpy().view(np.uint32), ws.view(np.uint32))


def test_topk_known_answers(dev):
    """tests/test_fg_vk.c:1274-1338."""
    import torch
    scores = np.array([1, 9, 7, 9, 3, 8, 2, 7, 6, 5, 4, 0, -1, -2, -3, -4, -5, -6, np.nan],
                      dtype=np.float32)
    ids = np.arange(19, dtype=np.uint32)
    ds, di = dev_f32(scores, dev), dev_u32(ids, dev)
    os_ = torch.empty(4, dtype=torch.float32, device=dev)
    oi = torch.empty(4, dtype=torch.int32, device=dev)
    for bad_k in (0, 65):
        with pytest.raises(fg_hip.FgStatusError) as e:
            fg_hip.topk_select(os_, oi, ds, di, 19, bad_k)
        assert e.value.code == fg_hip.FG_ERR_ARGUMENT
    assert fg_hip.topk_select(os_, oi, ds, di, 19, 4) == 4
    torch.cuda.synchronize()
    got_i, got_s = u32(oi), os_.cpu().numpy()
    assert sorted(got_i.tolist()) == [1, 2, 3, 5]
    assert np.array_equal(got_s, scores[got_i])
    first = (got_i.copy(), got_s.copy())
    fg_hip.topk_select(os_, oi, ds, di, 19, 4)
    torch.cuda.synchronize()
    assert np.array_equal(u32(oi), first[0]) and np.array_equal(os_.cpu().numpy(), first[1])
    assert fg_hip.topk_select(os_, oi, ds, di, 19, 1) == 1
    torch.cuda.synchronize()
    assert u32(oi)[0] == 1 and os_.cpu().numpy()[0] == 9.0  # tie 9.0 at ids 1, 3
    short = np.full(19, np.nan, dtype=np.float32)
    short[1], short[3] = 9.0, 8.0
    assert fg_hip.topk_select(os_, oi, dev_f32(short, dev), di, 19, 4) == 4
    torch.cuda.synchronize()
    gi, gs = u32(oi), os_.cpu().numpy()
    assert gi[0] != 0xFFFFFFFF and gi[1] != 0xFFFFFFFF and gi[2] == 0xFFFFFFFF
    assert not np.isfinite(gs[2])


@pytest.mark.parametrize("k", [1, 4, 20, 50, 64])
def test_topk_step_and_ladder_match_oracle(dev, k):
    import torch
    rng = np.random.default_rng(k)
    n = 151_936
    s = np.round(rng.normal(0, 3, n) * 4) / 4
    s = s.astype(np.float32)
    s[rng.integers(0, n, 100)] = np.nan
    s[rng.integers(0, n, 100)] = -np.inf
    s[5000:5100] = 0.0
    s[5100:5200] = -0.0
    tiles = (n + 1023) // 1024
    os_ = torch.empty(tiles * k, dtype=torch.float32, device=dev)
    oi = torch.empty(tiles * k, dtype=torch.int32, device=dev)
    ds = dev_f32(s, dev)
    produced = fg_hip.topk_select(os_, oi, ds, None, n, k)
    torch.cuda.synchronize()
    ws, wi = O.topk_select_step(s, k)
    assert produced == ws.size
    assert np.array_equal(u32(oi), wi)
    assert np.array_equal(os_.cpu().numpy().view(np.uint32), ws.view(np.uint32))
    # Ladder to a fixed point (src/output.c:681-700) = exact top-k by key.
    cur_s, cur_i, count = os_, oi, produced
    while count > k:
        t = (count + 1023) // 1024
        ns = torch.empty(t * k, dtype=torch.float32, device=dev)
        ni = torch.empty(t * k, dtype=torch.int32, device=dev)
        count = fg_hip.topk_select(ns, ni, cur_s, cur_i, count, k)
        cur_s, cur_i = ns, ni
    torch.cuda.synchronize()
    rs, ri, have = O.topk_row(s, k)
    assert sorted(u32(cur_i).tolist()) == sorted(ri.tolist())


def test_history_build_matches_oracle(dev):
    """fg_hip_history_build: Zipf histories with repeats against the oracle's
    tables (one launch, status per row on the device).  A row with an id
    outside the vocabulary reports FG_ERR_FORMAT and holds the counts of the
    ids before it (src/output.c:609-614 stops there); the other rows are
    unaffected.  The columns past vocab are never written."""
    import torch
    rows, vocab = 6, 151_936
    ids = O.gen_zipf_ids(rows, 1024, vocab, 1.1, 7, 7)
    want = O.build_counts(ids, vocab)
    d = torch.full((rows, vocab + 8), 123, dtype=torch.int32, device=dev)
    st = torch.full((rows,), -1, dtype=torch.int32, device=dev)
    offsets = torch.arange(0, (rows + 1) * 1024, 1024, dtype=torch.int64, device=dev)
    fg_hip.history_build(d, vocab + 8, vocab, dev_u32(ids.reshape(-1), dev), offsets, rows, st)
    torch.cuda.synchronize()
    got = u32(d)
    assert np.array_equal(got[:, :vocab], want)
    assert (got[:, vocab:] == 123).all()
    assert (st.cpu().numpy() == 0).all()
    bad = ids.copy()
    bad[2, 100] = vocab
    bad[2, 700] = vocab + 5
    bad[4, 0] = 0xFFFFFFFF
    fg_hip.history_build(d, vocab + 8, vocab, dev_u32(bad.reshape(-1), dev), offsets, rows, st)
    torch.cuda.synchronize()
    got = u32(d)
    assert st.cpu().numpy().tolist() == [0, 0, fg_hip.FG_ERR_FORMAT, 0, fg_hip.FG_ERR_FORMAT, 0]
    want_bad = want.copy()
    want_bad[2] = O.build_counts(ids[2:3, :100], vocab)[0]
    want_bad[4] = 0
    assert np.array_equal(got[:, :vocab], want_bad)


def test_history_build_on_two_streams(dev):
    """Two builds on two streams at once (different tables, statuses and id
    lists, one with a bad id): each reports only its own rows (no shared
    flag), and neither waits for the device."""
    import torch
    rows, vocab = 4, 151_936
    ids_a = O.gen_zipf_ids(rows, 2048, vocab, 1.1, 3, 3)
    ids_b = O.gen_zipf_ids(rows, 512, vocab, 1.1, 5, 5)
    ids_b[1, 17] = vocab
    outs = []
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    for ids, n, s in ((ids_a, 2048, streams[0]), (ids_b, 512, streams[1])):
        d = torch.zeros((rows, vocab), dtype=torch.int32, device=dev)
        st = torch.full((rows,), -1, dtype=torch.int32, device=dev)
        off = torch.arange(0, (rows + 1) * n, n, dtype=torch.int64, device=dev)
        dids = dev_u32(ids.reshape(-1), dev)
        torch.cuda.synchronize()
        fg_hip.history_build(d, vocab, vocab, dids, off, rows, st, stream=s.cuda_stream)
        outs.append((d, st, ids, dids, off))
    torch.cuda.synchronize()
    (da, sa, _, _, _), (db, sb, _, _, _) = outs
    assert (sa.cpu().numpy() == 0).all()
    assert sb.cpu().numpy().tolist() == [0, fg_hip.FG_ERR_FORMAT, 0, 0]
    assert np.array_equal(u32(da), O.build_counts(ids_a, vocab))
    want_b = O.build_counts(ids_b, vocab)
    want_b[1] = O.build_counts(ids_b[1:2, :17], vocab)[0]
    assert np.array_equal(u32(db), want_b)


@pytest.mark.parametrize("pad,extra", [(1, 5), (0, 8)])
def test_history_build_wire_matches_oracle(dev, pad, extra):
    """fg_hip_history_build_wire: valid payloads (Zipf histories with repeats,
    empty, one token, slot 1, aligned and unaligned starts) rebuild their
    rows; every malformation the decoder checks leaves its row's counts
    untouched and reports the decoder's status (oracle: the restated decoder,
    pinned to the reference's compiled codec).  pad shifts the blob (byte
    loads of the ids when odd, dword loads when payloads are 4-byte
    aligned); extra pads the row stride (16-byte stores of the counts when
    rows stay aligned)."""
    import struct
    import torch
    vocab = 151_936
    ids = O.gen_zipf_ids(3, 2000, vocab, 1.1, 9, 9)

    def wire(tokens, slot=0, count=None, reserved=b"\0\0\0"):
        n = len(tokens) if count is None else count
        return struct.pack(">IB", n, slot) + reserved + b"".join(struct.pack(">I", t) for t in tokens)

    payloads = [
        wire(ids[0].tolist()),                      # valid, many repeats
        wire([]),                                   # valid, empty
        wire([vocab - 1], slot=1),                  # valid, slot 1
        wire(ids[1].tolist()[:777]),                # valid (starts unaligned below)
        wire([1, 2, 3], slot=2),                    # bad slot
        wire([1, 2, 3], reserved=b"\0\0\1"),       # reserved byte
        wire([1, 2, 3], count=4),                   # count vs size
        wire([1, vocab, 3]),                        # token out of range
        b"\0\0\0",                                  # shorter than the header
        wire(ids[2].tolist()),                      # valid
    ]
    blob = bytearray(b"\x5a" * pad)                 # a pad byte: payload 0 starts unaligned
    offsets = []
    for pl in payloads:
        offsets.append(len(blob))
        blob += pl
    offsets.append(len(blob))
    rows = len(payloads)
    d_blob = torch.from_numpy(np.frombuffer(bytes(blob), dtype=np.uint8).copy()).to(dev)
    d_off = torch.tensor(offsets, dtype=torch.int64, device=dev)
    stride = vocab + extra
    counts = torch.full((rows, stride), 77, dtype=torch.int32, device=dev)
    status = torch.full((rows,), -1, dtype=torch.int32, device=dev)
    slots = torch.full((rows,), 9, dtype=torch.uint8, device=dev)
    fg_hip.history_build_wire(counts, stride, vocab, d_blob, d_off, rows, status, slots)
    torch.cuda.synchronize()
    got = u32(counts)
    st = status.cpu().numpy()
    sl = slots.cpu().numpy()
    for r, pl in enumerate(payloads):
        want_st, tokens, slot = O.history_decode(pl, 1 << 20, vocab)
        assert st[r] == want_st, f"row {r}: status {st[r]} vs {want_st}"
        if want_st == 0:
            want = np.bincount(np.asarray(tokens, dtype=np.int64), minlength=vocab).astype(np.uint32)
            assert np.array_equal(got[r, :vocab], want), f"row {r}: counts"
            assert sl[r] == slot
        else:
            assert (got[r, :vocab] == 77).all(), f"row {r}: counts changed"
        assert (got[r, vocab:] == 77).all()
    with pytest.raises(fg_hip.FgStatusError):
        fg_hip.history_build_wire(counts, vocab - 1, vocab, d_blob, d_off, rows, status)


def _reduce(dev, scores, ids):
    import torch
    n = scores.size
    cap = ((n + 4095) // 4096) * 512
    os_ = torch.empty(max(cap, 1), dtype=torch.float32, device=dev)
    oi = torch.empty(max(cap, 1), dtype=torch.int32, device=dev)
    got = fg_hip.topk_reduce(os_, oi, dev_f32(scores, dev),
                             None if ids is None else dev_u32(ids, dev), n)
    torch.cuda.synchronize()
    return os_.cpu().numpy()[:got], oi.cpu().numpy().view(np.uint32)[:got], got


def test_topk_reduce_reference_chunked():
    """tests/test_fg_vk.c:1231-1272 restated: the reference's LCG scores (with
    0, NaN, +Inf, -Inf every 97/257/389/521 entries), ids 0..count-1, its 39
    counts, and its checks (output count, each value equal to the input's at
    that id, comparator order within a tile, padding past the valid entries)."""
    import torch
    dev = torch.device("cuda:0")
    counts = [1, 2, 7, 63, 64, 65, 100, 127, 128, 129, 192, 320, 448, 511, 512, 513, 576, 640,
              704, 768, 1000, 1024, 1088, 1090, 1091, 1152, 1216, 2048, 2112, 3000, 4032, 4096,
              4097, 4160, 4224, 5000, 8000, 8192, 8200]
    mx = counts[-1]
    scores = np.empty(mx, dtype=np.float32)
    seed = 12345
    for i in range(mx):
        seed = (seed * 1664525 + 1013904223) & 0xFFFFFFFF
        v = np.float32(float(np.int32(np.uint32(seed >> 8)) % 2000) * 0.5)
        if i % 97 == 0:
            v = np.float32(0.0)
        if i % 257 == 0:
            v = np.float32(np.nan)
        if i % 389 == 0:
            v = np.float32(np.inf)
        if i % 521 == 0:
            v = np.float32(-np.inf)
        scores[i] = v
    ids = np.arange(mx, dtype=np.uint32)
    for count in counts:
        gs, gi, produced = _reduce(dev, scores[:count], ids[:count])
        tiles = (count + 4095) // 4096
        expected = count if tiles == 1 and count < 512 else tiles * 512
        assert produced == expected, count
        for i in range(produced):
            g, w = divmod(i, 512)
            remaining = max(count - g * 4096, 0)
            valid = min(remaining, 512)
            if w >= valid:
                assert gs[i] == -np.inf and gi[i] == 0xFFFFFFFF, (count, i)
            else:
                assert gi[i] < count and gs[i].view(np.uint32) == scores[gi[i]].view(np.uint32)
                if w + 1 < valid:
                    assert not O.reduce_before(gs[i + 1], gi[i + 1], gs[i], gi[i]), (count, i)


@pytest.mark.parametrize("count", [1, 511, 512, 4096, 4097, 20_000, 151_936])
def test_topk_reduce_matches_oracle(dev, count):
    """Bit-exact against the oracle's restatement: NaN payloads, +-Inf, +-0,
    quantised ties, arbitrary ids with some padding ids."""
    rng = np.random.default_rng(count)
    s = (np.round(rng.normal(0, 3, count) * 4) / 4).astype(np.float32)
    s[rng.random(count) < 0.01] = np.float32(np.nan)
    s.view(np.uint32)[rng.random(count) < 0.005] = 0x7FC00123  # NaN payload
    s[rng.random(count) < 0.005] = np.inf
    s[rng.random(count) < 0.005] = -np.inf
    s[rng.random(count) < 0.05] = -0.0
    ids = rng.permutation(count * 3)[:count].astype(np.uint32)
    ids[rng.random(count) < 0.01] = 0xFFFFFFFF
    gs, gi, produced = _reduce(dev, s, ids)
    ws, wi = O.topk_reduce_step(s, ids)
    assert produced == ws.size
    real = wi != 0xFFFFFFFF  # padding entries tie among themselves
    assert np.array_equal(gi[real], wi[real])
    assert np.array_equal(gs[real].view(np.uint32), ws[real].view(np.uint32))
    assert np.array_equal(gi == 0xFFFFFFFF, ~real)


def _reduce_tiles():
    """Tiles that take each route of the per-tile selection: the entries at
    positions p % 64 == 37 form its 64-entry sample (the kernel's layout),
    so a tile can place the sample where it wants it."""
    rng = np.random.default_rng(77)
    tiles = []
    for t in range(40):  # iid tiles: boundary buckets above and below 64 entries
        tiles.append(rng.normal(0, 1, 4096).astype(np.float32))
    samp = (np.arange(4096) % 64) == 37
    t = rng.normal(0, 1, 4096).astype(np.float32)  # sample = the tile's 64 largest
    t[samp] = np.sort(rng.normal(10, 1, 64)).astype(np.float32)
    tiles.append(t)
    t = rng.normal(0, 1, 4096).astype(np.float32)  # 8 huge, 56 below everything
    v = np.full(64, -50, dtype=np.float32)
    v[:8] = 50 + np.arange(8)
    t[samp] = rng.permutation(v)
    tiles.append(t)
    tiles.append(np.full(4096, 1.5, dtype=np.float32))  # all equal: ids decide
    tiles.append(np.sort(rng.normal(0, 1, 4096)).astype(np.float32))
    tiles.append(np.sort(rng.normal(0, 1, 4096))[::-1].astype(np.float32).copy())
    t = (np.round(rng.normal(0, 2, 4096)) / 2).astype(np.float32)  # few distinct values
    t[rng.random(4096) < 0.2] = np.nan
    tiles.append(t)
    t = rng.normal(0, 1, 4096).astype(np.float32)  # the top half of the sample tied
    t[samp] = np.where(np.arange(64) < 32, np.float32(3.0), t[samp])
    tiles.append(t)
    return np.concatenate(tiles)


@pytest.mark.parametrize("tail", [0, 1100, 3000])
def test_topk_reduce_selection_routes(dev, tail):
    """Every selection route of the tile kernel (all kept, a boundary of at
    most 64 entries, a boundary kept whole, later sample windows, the exact
    radix fallback) against the oracle, bit-exact; a partial last tile of
    `tail` entries; ids scattered with some padding ids."""
    rng = np.random.default_rng(5 + tail)
    s = _reduce_tiles()
    if tail:
        s = np.concatenate([s, rng.normal(0, 1, tail).astype(np.float32)])
    count = s.size
    ids = rng.permutation(count * 2)[:count].astype(np.uint32)
    ids[rng.random(count) < 0.002] = 0xFFFFFFFF
    gs, gi, produced = _reduce(dev, s, ids)
    ws, wi = O.topk_reduce_step(s, ids)
    assert produced == ws.size
    real = wi != 0xFFFFFFFF
    for g in range(produced // 512):
        sl = slice(g * 512, (g + 1) * 512)
        assert np.array_equal(gi[sl][real[sl]], wi[sl][real[sl]]), f"tile {g}"
        assert np.array_equal(gs[sl][real[sl]].view(np.uint32), ws[sl][real[sl]].view(np.uint32)), f"tile {g}"
    assert np.array_equal(gi == 0xFFFFFFFF, ~real)


def test_topk_reduce_ladder_gives_sorted_top512(dev):
    """Iterated as the reference's QSA scan iterates it (src/qsa.c:839-851):
    the final pass holds the global top-512 in comparator order."""
    import torch
    rng = np.random.default_rng(3)
    count = 300_000
    s = rng.normal(0, 1, count).astype(np.float32)
    s[rng.integers(0, count, 50)] = np.nan
    ids = np.arange(count, dtype=np.uint32)
    cur_s, cur_i, n = dev_f32(s, dev), dev_u32(ids, dev), count
    reduced = False
    while n > 512:
        cap = ((n + 4095) // 4096) * 512
        ns = torch.empty(cap, dtype=torch.float32, device=dev)
        ni = torch.empty(cap, dtype=torch.int32, device=dev)
        n = fg_hip.topk_reduce(ns, ni, cur_s, cur_i, n)
        cur_s, cur_i, reduced = ns, ni, True
    assert reduced and n == 512
    torch.cuda.synchronize()
    got = cur_i.cpu().numpy().view(np.uint32)[:512]
    want = np.lexsort(O.reduce_order_key(s, ids))[:512]
    assert np.array_equal(got, ids[want])


def _reduce_all(dev, scores, ids, work):
    import torch
    n = scores.size
    os_ = torch.full((512,), 7.0, dtype=torch.float32, device=dev)
    oi = torch.full((512,), 7, dtype=torch.int32, device=dev)
    got = fg_hip.topk_reduce_all(os_, oi, dev_f32(scores, dev),
                                 None if ids is None else dev_u32(ids, dev), n, work)
    torch.cuda.synchronize()
    return os_.cpu().numpy()[:got], oi.cpu().numpy().view(np.uint32)[:got], got


_REDUCE_ALL_ZEROED = 64 + 6 * 4096 * 4  # header and digit tables; the list is not read past its count


def _zeroed(work):
    """The counters and tables are zero after a call; bytes 4-7 and 16-19 hold
    the barrier generation and the call counter."""
    head = work[:_REDUCE_ALL_ZEROED].clone()
    head[4:8] = 0
    head[16:20] = 0
    return int(head.count_nonzero()) == 0


def _reduce_all_work(dev, count):
    import torch
    return torch.zeros(fg_hip.topk_reduce_all_workspace_bytes(count), dtype=torch.uint8, device=dev)


def _check_top(scores, ids, gs, gi, got):
    """The first min(count, 512) entries in comparator order (padding ids,
    which tie among themselves, compared as a set)."""
    want = np.lexsort(O.reduce_order_key(scores, ids))[:min(scores.size, 512)]
    assert got == want.size
    wi, ws = ids[want], scores[want]
    real = wi != 0xFFFFFFFF
    assert np.array_equal(gi[real], wi[real])
    assert np.array_equal(gs[real].view(np.uint32), ws[real].view(np.uint32))
    assert np.array_equal(gi == 0xFFFFFFFF, ~real)


def test_topk_reduce_all_matches_the_ladder(dev):
    """One launch against the per-level ladder it replaces (src/qsa.c:839-851)
    on the same 300,000 scores with NaNs: the same 512 entries in the same
    order, bit-exact."""
    import torch
    rng = np.random.default_rng(3)
    count = 300_000
    s = rng.normal(0, 1, count).astype(np.float32)
    s[rng.integers(0, count, 50)] = np.nan
    ids = np.arange(count, dtype=np.uint32)
    cur_s, cur_i, n = dev_f32(s, dev), dev_u32(ids, dev), count
    while n > 512:
        cap = ((n + 4095) // 4096) * 512
        ns = torch.empty(cap, dtype=torch.float32, device=dev)
        ni = torch.empty(cap, dtype=torch.int32, device=dev)
        n = fg_hip.topk_reduce(ns, ni, cur_s, cur_i, n)
        cur_s, cur_i = ns, ni
    work = _reduce_all_work(dev, count)
    gs, gi, got = _reduce_all(dev, s, None, work)
    assert got == 512
    assert np.array_equal(gi, cur_i.cpu().numpy().view(np.uint32)[:512])
    assert np.array_equal(gs.view(np.uint32), cur_s.cpu().numpy()[:512].view(np.uint32))
    _check_top(s, ids, gs, gi, got)
    assert _zeroed(work), "workspace not returned to zero"


@pytest.mark.parametrize("count", [1, 7, 511, 512, 513, 4096, 4097, 20_000, 151_936, 262_144])
def test_topk_reduce_all_matches_oracle(dev, count):
    """NaN payloads, +-Inf, quantised ties, scattered ids with some padding
    ids, partial last tiles and counts under 512; one workspace reused by
    two calls, the second smaller."""
    rng = np.random.default_rng(count + 1)
    work = _reduce_all_work(dev, count)
    for n in (count, max(1, count // 3)):
        s = (np.round(rng.normal(0, 3, n) * 4) / 4).astype(np.float32)
        s[rng.random(n) < 0.01] = np.float32(np.nan)
        s.view(np.uint32)[rng.random(n) < 0.005] = 0x7FC00123
        s[rng.random(n) < 0.005] = np.inf
        s[rng.random(n) < 0.005] = -np.inf
        ids = rng.permutation(n * 3)[:n].astype(np.uint32)
        ids[rng.random(n) < 0.01] = 0xFFFFFFFF
        gs, gi, got = _reduce_all(dev, s, ids, work)
        _check_top(s, ids, gs, gi, got)
    assert _zeroed(work)


@pytest.mark.parametrize("kind", ["equal", "duplicate_ids", "sorted", "one_tile_high"])
def test_topk_reduce_all_adversarial(dev, kind):
    """Inputs that defeat the tile bounds: every score equal (ids decide),
    entries repeated with the same id, ascending scores (the last tile holds
    the whole answer), one tile far above the rest."""
    rng = np.random.default_rng(11)
    count = 100_000
    ids = np.arange(count, dtype=np.uint32)
    if kind == "equal":
        s = np.full(count, 2.5, dtype=np.float32)
        ids = rng.permutation(count).astype(np.uint32)
    elif kind == "duplicate_ids":
        s = (np.round(rng.normal(0, 1, count)) + 0.5).astype(np.float32)
        ids = rng.integers(0, 700, count).astype(np.uint32)
    elif kind == "sorted":
        s = np.sort(rng.normal(0, 1, count)).astype(np.float32)
    else:
        s = rng.normal(0, 1, count).astype(np.float32)
        s[8192:12288] += 100
    work = _reduce_all_work(dev, count)
    gs, gi, got = _reduce_all(dev, s, ids, work)
    if kind == "duplicate_ids":
        # identical (score, id) entries tie: compare the ordered pairs
        want = np.lexsort(O.reduce_order_key(s, ids))[:512]
        assert got == 512
        assert np.array_equal(gi, ids[want])
        assert np.array_equal(gs, s[want])
    else:
        _check_top(s, ids, gs, gi, got)
    assert _zeroed(work)


def test_topk_reduce_all_limits(dev):
    import torch
    x = torch.zeros(8, device=dev)
    w = torch.zeros(256, dtype=torch.uint8, device=dev)
    with pytest.raises(fg_hip.FgStatusError) as e:
        fg_hip.topk_reduce_all(x, x, x, None, 0, w)
    assert e.value.code == fg_hip.FG_ERR_ARGUMENT
    big = 1 << 26  # 16,384 tiles: more workgroups than the device holds at once
    with pytest.raises(fg_hip.FgStatusError) as e:
        fg_hip.topk_reduce_all(x, x, x, None, big, w)
    assert e.value.code == fg_hip.FG_ERR_LIMIT


def test_topk_reduce_argument_errors(dev):
    import torch
    x = torch.zeros(8, device=dev)
    with pytest.raises(fg_hip.FgStatusError) as e:
        fg_hip.topk_reduce(x, x, x, None, 0)
    assert e.value.code == fg_hip.FG_ERR_ARGUMENT
