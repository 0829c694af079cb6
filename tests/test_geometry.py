"""Launch geometry of the batched sampler, on the host (no device): the
chunking rule, the wave slices and the workgroup -> (row, chunk) layout that
the kernel itself uses (fg_sampler_hip_plan / fg_sampler_hip_block call the
same host-device functions as the kernel).

Properties: every (row, chunk) is taken by exactly one workgroup; a row's
wave slices tile [0, vocab) in order, each a multiple of 4 elements except
the one that ends the row; a row's chunks share one residue of the
workgroup index mod 8 (one XCD under the round-robin dispatch) when the row
count is a multiple of 8; in the paired layout a row's first `split` chunks
run in the grid's first half."""
import pytest

import fg_hip

V = 151_936
NUC, UNLIKE = fg_hip.ROWS_NUCLEUS, fg_hip.ROWS_UNLIKE_COST


def layout(vocab, rows, g):
    seen = {}
    slices = {}
    for b in range(rows * g.chunks):
        for w in range(4):
            row, chunk, begin, end = fg_hip.block(g, vocab, rows, b, w)
            if w == 0:
                assert (row, chunk) not in seen, f"block {b} repeats {(row, chunk)}"
                seen[(row, chunk)] = b
            slices.setdefault(row, []).append((chunk * 4 + w, begin, end))
    assert len(seen) == rows * g.chunks
    return seen, slices


def check_geometry(vocab, rows, g, groups_cap):
    assert 1 <= g.chunks <= 64
    assert rows * g.chunks <= groups_cap + rows
    assert g.split <= g.chunks and g.wave_elems % 4 == 0 and g.wave_elems_b % 4 == 0
    seen, slices = layout(vocab, rows, g)
    for row in range(rows):
        at = 0
        for i, begin, end in sorted(slices[row]):
            assert begin == at, f"row {row} wave {i}: starts at {begin}, expected {at}"
            assert end >= begin
            assert (end - begin) % 4 == 0 or end == vocab
            at = end
        assert at == vocab, f"row {row} covers [0, {at}) of {vocab}"
        if rows % 8 == 0:
            assert len({seen[(row, c)] % 8 for c in range(g.chunks)}) == 1
        if g.split < g.chunks:
            half = rows * g.split
            for c in range(g.chunks):
                assert (seen[(row, c)] < half) == (c < g.split)


@pytest.mark.parametrize("vocab,rows,traits", [
    (V, 64, 0), (V, 256, NUC), (V, 128, UNLIKE), (V, 1024, 0), (V, 1, 0), (V, 12, 0),
    (V, 48, UNLIKE), (V, 256, 0), (3001, 8, 0), (5, 3, 0), (1, 1, 0), (65_537, 16, NUC),
    (262_144, 32, 0), (1000, 8, 0)])
def test_rule_geometry(monkeypatch, vocab, rows, traits):
    for name in ("FG_HIP_TARGET_GROUPS", "FG_HIP_PAIRED", "FG_HIP_FRONT_SHARE", "FG_HIP_PACE"):
        monkeypatch.delenv(name, raising=False)
    g = fg_hip.plan(vocab, rows, traits)
    check_geometry(vocab, rows, g, 1024)
    assert g.pace == 1


@pytest.mark.parametrize("groups,share,paired", [(32, 650, 1), (128, 600, 1), (128, 0, 0),
                                                 (2048, 0, 1), (16, 749, 1)])
def test_override_geometry(monkeypatch, groups, share, paired):
    monkeypatch.setenv("FG_HIP_TARGET_GROUPS", str(groups))
    monkeypatch.setenv("FG_HIP_PAIRED", str(paired))
    if share:
        monkeypatch.setenv("FG_HIP_FRONT_SHARE", str(share))
    monkeypatch.setenv("FG_HIP_PACE", "0")
    g = fg_hip.plan(V, 16)
    check_geometry(V, 16, g, max(groups, 1024))
    assert g.pace == 0
    if paired and g.chunks % 2 == 0:
        assert g.split == g.chunks // 2
        if share > 500:
            assert g.wave_elems > g.wave_elems_b


def test_benchmark_rules(monkeypatch):
    """The rule's choices for the benchmark configurations (measured on
    MI355X): config 2 paired, 8 chunks, longer first-half slices; config 3 (nucleus) 3
    chunks; config 4 (unlike rows) 4 chunks row-major; config 5 one chunk."""
    for name in ("FG_HIP_TARGET_GROUPS", "FG_HIP_PAIRED", "FG_HIP_FRONT_SHARE", "FG_HIP_PACE"):
        monkeypatch.delenv(name, raising=False)
    g = fg_hip.plan(V, 64)
    assert (g.chunks, g.split) == (8, 4) and g.wave_elems > g.wave_elems_b
    g = fg_hip.plan(V, 256, NUC)
    assert (g.chunks, g.split) == (3, 3)
    g = fg_hip.plan(V, 128, UNLIKE)
    assert (g.chunks, g.split) == (4, 4)
    g = fg_hip.plan(V, 1024)
    assert g.chunks == 1


def test_argument_errors():
    g = fg_hip.plan(V, 64)
    with pytest.raises(Exception):
        fg_hip.plan(0, 64)
    with pytest.raises(Exception):
        fg_hip.plan(V, 0)
    with pytest.raises(Exception):
        fg_hip.plan(V, 64, 4)
    with pytest.raises(Exception):
        fg_hip.block(g, V, 64, 64 * g.chunks, 0)
    with pytest.raises(Exception):
        fg_hip.block(g, V, 64, 0, 4)
