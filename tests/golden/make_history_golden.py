"""Writes tests/golden/ref_history_vectors.json from the reference's own
output-history codec, compiled from its sources by `make -C oracle ref` into
oracle/_ref/libfg_ref_protocol.so (reference src/protocol.c with the four
sources it links against).

The vectors pin, on fixed inputs, what the reference computes:
  * fg_output_history_encode (src/protocol.c:1328-1346): status and payload
    bytes for valid histories, empty ones, out-of-vocabulary tokens, bad
    session slots, too-small capacities;
  * fg_output_history_decode (src/protocol.c:1348-1366): status, tokens and
    slot for valid payloads and for every malformation the decoder checks
    (short header, reserved bytes, slot, count vs size, count vs capacity,
    token range).
The reference's vocabulary is FG_Q38_VOCAB_SIZE (248,320).
Run in the build container (where /root/reference exists):
    python tests/golden/make_history_golden.py
"""
from __future__ import annotations

import ctypes as C
import json
import struct
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
LIB = ROOT / "oracle" / "_ref" / "libfg_ref_protocol.so"
OUT = Path(__file__).resolve().parent / "ref_history_vectors.json"
V = 248320


class RefError(C.Structure):
    _fields_ = [("code", C.c_int), ("message", C.c_char * 512)]


class RefHistory(C.Structure):
    _fields_ = [("tokens", C.c_void_p), ("count", C.c_uint32), ("session_slot", C.c_uint8)]


def encode(lib, tokens, slot, capacity):
    t = np.asarray(tokens, dtype=np.uint32)
    h = RefHistory(t.ctypes.data if t.size else None, t.size, slot)
    buf = (C.c_uint8 * max(capacity, 1))()
    n = C.c_uint32(0)
    err = RefError()
    st = lib.fg_output_history_encode(buf, capacity, C.byref(n), C.byref(h), C.byref(err))
    return dict(status=int(st), payload=bytes(buf[:n.value]).hex() if st == 0 else None)


def decode(lib, payload: bytes, capacity):
    storage = np.zeros(max(capacity, 1), dtype=np.uint32)
    h = RefHistory()
    src = (C.c_uint8 * max(len(payload), 1)).from_buffer_copy(payload or b"\0")
    err = RefError()
    st = lib.fg_output_history_decode(C.byref(h), storage.ctypes.data if capacity else None,
                                      capacity, src, len(payload), C.byref(err))
    ok = st == 0
    return dict(status=int(st), tokens=storage[:h.count].tolist() if ok else None,
                slot=int(h.session_slot) if ok else None)


def main():
    if not LIB.exists():
        sys.exit(f"{LIB} is missing: run `make -C oracle ref` first")
    lib = C.CDLL(str(LIB))
    P, E, H, u32 = C.c_void_p, C.POINTER(RefError), C.POINTER(RefHistory), C.c_uint32
    lib.fg_output_history_encode.argtypes = [P, u32, C.POINTER(u32), H, E]
    lib.fg_output_history_decode.argtypes = [H, P, u32, P, u32, E]
    rng = np.random.default_rng(20261202)
    enc, dec = [], []
    # Encode: the reference test's {7, 7, 42} (tests/test_core.c:944-950), empty,
    # random lengths, slot 1, bad slot, vocab edge, capacity edges.
    cases = [([7, 7, 42], 0, 64), ([], 0, 64), ([V - 1, 0, 1], 1, 64), ([V], 0, 64),
             ([1, 2, 3], 2, 64), ([1, 2, 3], 1, 19), ([1, 2, 3], 1, 20), ([], 0, 7)]
    for n in (1, 5, 64, 1000):
        cases.append((rng.integers(0, V, n).tolist(), int(rng.integers(0, 2)), 8 + 4 * n))
    for tokens, slot, cap in cases:
        enc.append(dict(tokens=tokens, slot=slot, capacity=cap, **encode(lib, tokens, slot, cap)))
    # Decode: valid payloads, then every malformation.
    def payload(count, slot, reserved=(0, 0, 0), tokens=()):
        return struct.pack(">IB3B", count, slot, *reserved) + b"".join(
            struct.pack(">I", t) for t in tokens)
    good = payload(3, 0, tokens=(7, 7, 42))
    dcases = [(good, 8), (payload(0, 0), 0), (payload(0, 1), 4), (good, 3), (good, 2),
              (payload(3, 2, tokens=(7, 7, 42)), 8), (payload(3, 0, (0, 0, 1), (7, 7, 42)), 8),
              (payload(3, 0, (1, 0, 0), (7, 7, 42)), 8), (good[:-1], 8), (good + b"\0", 8),
              (good[:7], 8), (b"", 8), (payload(4, 0, tokens=(7, 7, 42)), 8),
              (payload(2, 1, tokens=(V - 1, 0)), 8), (payload(2, 1, tokens=(V, 0)), 8),
              (payload(1, 0, tokens=(0xffffffff,)), 8), (payload(262145, 0), 300000)]
    for n in (1, 17, 500):
        t = rng.integers(0, V, n).tolist()
        dcases.append((payload(n, int(rng.integers(0, 2)), tokens=t), n))
    for data, cap in dcases:
        dec.append(dict(payload=data.hex(), capacity=cap, **decode(lib, data, cap)))
    doc = dict(source="reference src/protocol.c (+ util.c, sampler.c, topology.c, sha256.c) "
                      "compiled by oracle/Makefile (ref)", vocab=V, encode=enc, decode=dec)
    OUT.write_text(json.dumps(doc, separators=(",", ":")))
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes): {len(enc)} encode, {len(dec)} decode")


if __name__ == "__main__":
    main()
