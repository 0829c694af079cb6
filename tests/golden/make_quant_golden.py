"""Writes tests/golden/ref_quant_vectors.json from the reference's own Q8_0
code (src/quant.c), compiled from its sources by `make -C oracle ref` into
oracle/_ref/libfg_ref_quant.so:
  * fg_f16_to_f32 over all 65,536 inputs (SHA-256 of the f32 table);
  * fg_f32_to_f16 over a structured set of 2^20 binary32 patterns (every
    exponent and sign, mantissas at and around each rounding boundary and
    seeded random ones; SHA-256 of the u16 table) plus named edge cases;
  * fg_quantize_q8_0 on seeded inputs with ties, zero blocks, huge and tiny
    magnitudes (output bytes, hex for small cases, SHA-256 for large);
  * fg_q8_0_cooked_tile_bytes / _matrix_bytes on a grid of shapes;
  * fg_cook_q8_0_rows on seeded packed matrices (SHA-256 of the cooked bytes).
Run in the build container (where /root/reference exists):
    python tests/golden/make_quant_golden.py
"""
from __future__ import annotations

import ctypes as C
import hashlib
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
LIB = ROOT / "oracle" / "_ref" / "libfg_ref_quant.so"
OUT = Path(__file__).resolve().parent / "ref_quant_vectors.json"
sys.path.insert(0, str(Path(__file__).resolve().parent.parent))
import quant_inputs as QI  # noqa: E402


def bind(lib):
    u32, u64, P = C.c_uint32, C.c_uint64, C.c_void_p
    lib.fg_f16_to_f32.argtypes, lib.fg_f16_to_f32.restype = [C.c_uint16], C.c_float
    lib.fg_f32_to_f16.argtypes, lib.fg_f32_to_f16.restype = [C.c_float], C.c_uint16
    lib.fg_quantize_q8_0.argtypes, lib.fg_quantize_q8_0.restype = [P, P, u64], None
    lib.fg_q8_0_cooked_tile_bytes.argtypes, lib.fg_q8_0_cooked_tile_bytes.restype = [u32], u64
    lib.fg_q8_0_cooked_matrix_bytes.argtypes = [u32, u32]
    lib.fg_q8_0_cooked_matrix_bytes.restype = u64
    lib.fg_cook_q8_0_rows.argtypes, lib.fg_cook_q8_0_rows.restype = [P, P, u64, u32, u32], C.c_bool
    return lib


def main():
    if not LIB.exists():
        sys.exit(f"{LIB} is missing: run `make -C oracle ref` first")
    lib = bind(C.CDLL(str(LIB)))
    doc = {"source": "reference src/quant.c compiled by oracle/Makefile (ref)"}
    f32 = np.array([lib.fg_f16_to_f32(h) for h in range(65536)], dtype=np.float32)
    doc["f16_to_f32_sha256"] = hashlib.sha256(f32.tobytes()).hexdigest()
    pats = QI.f32_patterns()
    f16 = np.array([lib.fg_f32_to_f16(C.c_float(v)) for v in pats.view(np.float32)],
                   dtype=np.uint16)
    doc["f32_to_f16_sha256"] = hashlib.sha256(f16.tobytes()).hexdigest()
    doc["f32_to_f16_cases"] = [[int(u), int(lib.fg_f32_to_f16(C.c_float(np.uint32(u).view(np.float32))))]
                               for u in QI.F32_EDGES]
    quant = []
    for name, x in QI.quant_cases():
        out = np.zeros(x.size // 32 * 34, dtype=np.uint8)
        lib.fg_quantize_q8_0(x.ctypes.data, out.ctypes.data, x.size)
        quant.append({"name": name, "sha256": hashlib.sha256(out.tobytes()).hexdigest(),
                      "hex": out.tobytes().hex() if out.size <= 340 else None})
    doc["quantize"] = quant
    doc["sizes"] = [[w, r, int(lib.fg_q8_0_cooked_tile_bytes(w)),
                     int(lib.fg_q8_0_cooked_matrix_bytes(w, r))]
                    for w in QI.SIZE_WIDTHS for r in QI.SIZE_ROWS]
    cook = []
    for w, r, packed in QI.cook_cases():
        n = int(lib.fg_q8_0_cooked_matrix_bytes(w, r))
        out = np.full(n, 0xAB, dtype=np.uint8)
        short = bool(lib.fg_cook_q8_0_rows(packed.ctypes.data, out.ctypes.data, n - 1, w, r))
        ok = bool(lib.fg_cook_q8_0_rows(packed.ctypes.data, out.ctypes.data, n, w, r))
        cook.append({"width": w, "rows": r, "ok": ok, "short_ok": short,
                     "sha256": hashlib.sha256(out.tobytes()).hexdigest()})
    doc["cook"] = cook
    OUT.write_text(json.dumps(doc, separators=(",", ":")))
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
