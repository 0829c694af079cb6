"""Seeded inputs shared by tests/golden/make_quant_golden.py (which records
the reference's outputs on them) and tests/test_quant.py (which checks this
build's Q8_0 code on the same inputs)."""
import numpy as np

F32_EDGES = [0x00000000, 0x80000000, 0x7f800000, 0xff800000, 0x7fc00000, 0xffc00001,
             0x7f800001, 0x477fe000, 0x477fefff, 0x477ff000, 0x477fffff, 0x47800000,
             0x38800000, 0x387fffff, 0x33800000, 0x33800001, 0x33000000, 0x33000001,
             0x32ffffff, 0x3f800000, 0x3f801000, 0x3f803000, 0x3f801001, 0x00000001,
             0x3c000000 + 0x1000, 0x3c002000 + 0x1000, 0xc77fefff]
SIZE_WIDTHS = [0, 1, 31, 32, 33, 64, 320, 2560, 4096, 65536]
SIZE_ROWS = [0, 1, 15, 16, 17, 248320]


def f32_patterns() -> np.ndarray:
    """2^20 binary32 bit patterns: each (sign, exponent) with mantissas at and
    around every binary16 rounding boundary plus seeded random mantissas."""
    rng = np.random.default_rng(16)
    out = []
    for sign in (0, 1):
        for e in range(256):
            base = (sign << 31) | (e << 23)
            m = np.concatenate([
                np.arange(0, 1 << 23, 1 << 13, dtype=np.uint32)[:512],          # exact halves
                (np.arange(0, 512, dtype=np.uint32) << 13) + (1 << 12),        # ties
                (np.arange(0, 512, dtype=np.uint32) << 13) + (1 << 12) - 1,
                (np.arange(0, 512, dtype=np.uint32) << 13) + (1 << 12) + 1,
            ])
            m = np.concatenate([m, rng.integers(0, 1 << 23, 2048 - m.size, dtype=np.uint32)])
            out.append(np.uint32(base) | (m & np.uint32(0x7fffff)))
    return np.concatenate(out).astype(np.uint32)


def quant_cases():
    rng = np.random.default_rng(8)
    yield "normal", rng.normal(0, 1, 32 * 64).astype(np.float32)
    yield "small", rng.normal(0, 1e-6, 32 * 8).astype(np.float32)
    yield "huge", (rng.normal(0, 1, 32 * 8) * 1e30).astype(np.float32)
    z = rng.normal(0, 1, 32 * 4).astype(np.float32)
    z[32:64] = 0.0
    z[64:96] = -0.0
    yield "zero_blocks", z
    t = np.tile(np.array([127, -127, 63.5, -63.5, 0.5, -0.5, 1.5, 2.5] * 4, np.float32), 4)
    yield "ties", t
    u = rng.normal(0, 1, 32 * 16).astype(np.float32)
    u[::7] = np.float32(65504.0 * 127)  # d overflows binary16
    yield "scale_overflow", u
    yield "subnormal_scale", (rng.normal(0, 1, 32 * 8) * 1e-9).astype(np.float32)
    yield "large_matrix", rng.normal(0, 0.02, 32 * 80 * 40).astype(np.float32)


def cook_cases():
    rng = np.random.default_rng(96)
    for w, r in ((32, 1), (320, 2), (320, 17), (64, 33), (2560, 16), (2560, 19)):
        packed = rng.integers(0, 256, (w // 32) * 34 * r, dtype=np.uint8)
        yield w, r, packed
