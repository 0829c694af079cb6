"""Writes tests/golden/ref_split_layout.json from the reference's own
vocabulary-split layout functions, compiled from its sources by
`make -C oracle ref` into oracle/_ref/libfg_ref_protocol.so:
  * fg_output_split_way_for_rank (src/protocol.c:23-37) for ways 0..5, ranks 0..8;
  * fg_output_split_rank (src/protocol.c:39-44) for ways 0..5, ways 0..5;
  * fg_output_split_span (src/protocol.c:93-105) for ways 0..5, ways 0..5.
Run in the build container (where /root/reference exists):
    python tests/golden/make_split_golden.py
"""
from __future__ import annotations

import ctypes as C
import json
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
LIB = ROOT / "oracle" / "_ref" / "libfg_ref_protocol.so"
OUT = Path(__file__).resolve().parent / "ref_split_layout.json"


def main():
    if not LIB.exists():
        sys.exit(f"{LIB} is missing: run `make -C oracle ref` first")
    lib = C.CDLL(str(LIB))
    u32 = C.c_uint32
    lib.fg_output_split_way_for_rank.argtypes = [u32, u32, C.POINTER(u32)]
    lib.fg_output_split_way_for_rank.restype = C.c_bool
    lib.fg_output_split_rank.argtypes = [u32, u32]
    lib.fg_output_split_rank.restype = u32
    lib.fg_output_split_span.argtypes = [u32, u32, C.POINTER(u32), C.POINTER(u32)]
    lib.fg_output_split_span.restype = None
    way_for_rank, rank, span = [], [], []
    for ways in range(6):
        for r in range(9):
            w = u32(0xDEAD)
            ok = bool(lib.fg_output_split_way_for_rank(ways, r, C.byref(w)))
            way_for_rank.append([ways, r, ok, w.value if ok else None])
        for way in range(6):
            rank.append([ways, way, int(lib.fg_output_split_rank(ways, way))])
            first, rows = u32(7), u32(7)
            lib.fg_output_split_span(ways, way, C.byref(first), C.byref(rows))
            span.append([ways, way, first.value, rows.value])
    doc = dict(source="reference src/protocol.c compiled by oracle/Makefile (ref)",
               way_for_rank=way_for_rank, rank=rank, span=span)
    OUT.write_text(json.dumps(doc, separators=(",", ":")))
    print(f"wrote {OUT}: {len(way_for_rank)} way_for_rank, {len(rank)} rank, {len(span)} span")


if __name__ == "__main__":
    main()
