"""Q8_0 host code (include/fg_quant.h) against the reference's compiled
src/quant.c (tests/golden/ref_quant_vectors.json), the reference's own
cooking test (tests/test_core.c:846-870) restated, and properties: binary16
conversions against numpy's IEEE ones, uncook(cook(x)) = x."""
import ctypes as C
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

import fg_hip
import quant_inputs as QI

G = json.loads((Path(__file__).parent / "golden" / "ref_quant_vectors.json").read_text())


def lib():
    return fg_hip.lib()


def test_f16_to_f32_all_inputs():
    t = np.array([lib().fg_f16_to_f32(h) for h in range(65536)], dtype=np.float32)
    assert hashlib.sha256(t.tobytes()).hexdigest() == G["f16_to_f32_sha256"]
    finite = np.arange(65536, dtype=np.uint16)
    ok = (finite & 0x7c00) != 0x7c00
    assert np.array_equal(t[ok], finite[ok].view(np.float16).astype(np.float32))


def test_f32_to_f16_structured_set():
    pats = QI.f32_patterns()
    f = pats.view(np.float32)
    got = np.array([lib().fg_f32_to_f16(C.c_float(v)) for v in f], dtype=np.uint16)
    assert hashlib.sha256(got.tobytes()).hexdigest() == G["f32_to_f16_sha256"]
    ok = np.isfinite(f)
    with np.errstate(over="ignore"):
        assert np.array_equal(got[ok], f[ok].astype(np.float16).view(np.uint16))  # IEEE RNE
    for u, want in G["f32_to_f16_cases"]:
        assert lib().fg_f32_to_f16(C.c_float(np.uint32(u).view(np.float32))) == want, hex(u)


@pytest.mark.parametrize("case", range(8))
def test_quantize_matches_reference(case):
    name, x = list(QI.quant_cases())[case]
    want = G["quantize"][case]
    assert want["name"] == name
    out = fg_hip.quantize_q8_0(x)
    assert hashlib.sha256(out.tobytes()).hexdigest() == want["sha256"]
    if want["hex"] is not None:
        assert out.tobytes().hex() == want["hex"]


def test_dequantize_is_scale_times_quant():
    x = np.random.default_rng(1).normal(0, 1, 32 * 10).astype(np.float32)
    packed = fg_hip.quantize_q8_0(x)
    out = np.empty(x.size, dtype=np.float32)
    lib().fg_dequantize_q8_0(packed.ctypes.data, out.ctypes.data, x.size)
    b = packed.reshape(10, 34)
    d = b[:, :2].copy().view(np.float16).astype(np.float32)
    q = b[:, 2:].view(np.int8).astype(np.float32)
    assert np.array_equal(out.reshape(10, 32), d * q)
    # q rounds x / d32; the stored scale is d32 rounded to binary16, which
    # moves d*q by at most 127 * |d| * 2^-11 more.
    assert np.all(np.abs(out - x).reshape(10, 32) <= np.abs(d) * (0.5 + 127 * 2.0**-11) + 1e-7)


def test_cooked_sizes_match_reference():
    for w, r, tile, matrix in G["sizes"]:
        assert lib().fg_q8_0_cooked_tile_bytes(w) == tile, (w, r)
        assert lib().fg_q8_0_cooked_matrix_bytes(w, r) == matrix, (w, r)


def test_cook_matches_reference_and_round_trips():
    for (w, r, packed), want in zip(QI.cook_cases(), G["cook"]):
        assert (w, r) == (want["width"], want["rows"])
        n = lib().fg_q8_0_cooked_matrix_bytes(w, r)
        out = np.full(n, 0xAB, dtype=np.uint8)
        assert lib().fg_cook_q8_0_rows(packed.ctypes.data, out.ctypes.data, n - 1, w, r) == want["short_ok"]
        assert lib().fg_cook_q8_0_rows(packed.ctypes.data, out.ctypes.data, n, w, r) == want["ok"]
        assert hashlib.sha256(out.tobytes()).hexdigest() == want["sha256"]
        back = np.zeros(packed.size, dtype=np.uint8)
        assert lib().fg_uncook_q8_0_rows(out.ctypes.data, back.ctypes.data, back.size, w, r)
        assert np.array_equal(back, packed)


def test_cook_reference_layout_test():
    """tests/test_core.c:846-870 restated: width 320, 2 rows."""
    width, rows, blocks = 320, 2, 10
    tile_bytes, quant_offset = 16 * blocks * 34, 16 * blocks * 2
    packed = np.zeros(rows * blocks * 34, dtype=np.uint8)
    for row in range(rows):
        for block in range(blocks):
            src = (row * blocks + block) * 34
            s = lib().fg_f32_to_f16(C.c_float(0.25 + (row * blocks + block) * 0.03125))
            packed[src:src + 2] = [s & 0xFF, s >> 8]
            packed[src + 2:src + 34] = [(row * 73 + block * 31 + i * 7) & 0xFF for i in range(32)]
    assert lib().fg_q8_0_cooked_tile_bytes(width) == tile_bytes
    assert lib().fg_q8_0_cooked_matrix_bytes(width, rows) == tile_bytes
    cooked = np.zeros(tile_bytes, dtype=np.uint8)
    assert lib().fg_cook_q8_0_rows(packed.ctypes.data, cooked.ctypes.data, tile_bytes, width, rows)
    for row in range(rows):
        for block in range(blocks):
            src = (row * blocks + block) * 34
            at = (block * 16 + row) * 2
            assert np.array_equal(cooked[at:at + 2], packed[src:src + 2])
            q = quant_offset + (row * blocks + block) * 32
            assert np.array_equal(cooked[q:q + 32], packed[src + 2:src + 34])
    for block in range(blocks):
        for row in range(rows, 16):
            assert cooked[(block * 16 + row) * 2] == 0
    assert not lib().fg_cook_q8_0_rows(packed.ctypes.data, cooked.ctypes.data, tile_bytes - 1,
                                       width, rows)
