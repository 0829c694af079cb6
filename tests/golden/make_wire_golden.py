"""Writes tests/golden/ref_output_wire_vectors.json from the reference's own
output-owner wire codecs, compiled from its sources by `make -C oracle ref`
into oracle/_ref/libfg_ref_protocol.so:
  * fg_output_config_encode / fg_output_config_decode (src/protocol.c:1160-1166);
  * fg_output_result_encode / fg_output_result_decode (src/protocol.c:1275-1279).
Inputs: valid configs and results, every route / sampler / draw check failing
once, and payloads mutated byte by byte (sizes, flags, reserved bytes).
Run in the build container (where /root/reference exists):
    python tests/golden/make_wire_golden.py
"""
from __future__ import annotations

import ctypes as C
import json
import math
import struct
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
LIB = ROOT / "oracle" / "_ref" / "libfg_ref_protocol.so"
OUT = Path(__file__).resolve().parent / "ref_output_wire_vectors.json"


class Sampler(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("top_k", C.c_uint32),
                ("presence_penalty", C.c_float), ("frequency_penalty", C.c_float),
                ("repetition_penalty", C.c_float), ("min_p", C.c_float), ("seed", C.c_uint64)]


class Config(C.Structure):
    _fields_ = [("source_rank", C.c_uint8), ("destination_rank", C.c_uint8),
                ("flags", C.c_uint8), ("session_slot", C.c_uint8), ("token_index", C.c_uint32),
                ("sampler", Sampler), ("uniform", C.c_float)]


class Result(C.Structure):
    _fields_ = [("source_rank", C.c_uint8), ("destination_rank", C.c_uint8),
                ("token_index", C.c_uint32), ("token", C.c_uint32), ("logit", C.c_float)]


class Err(C.Structure):
    _fields_ = [("code", C.c_int), ("message", C.c_char * 512)]


SAMPLER_FIELDS = ("temperature", "top_p", "top_k", "presence_penalty", "frequency_penalty",
                  "repetition_penalty", "min_p")


def f32_bits(x):
    return struct.unpack("<I", struct.pack("<f", x))[0]


def config_dict(c):
    return {"source_rank": c.source_rank, "destination_rank": c.destination_rank,
            "flags": c.flags, "session_slot": c.session_slot, "token_index": c.token_index,
            "sampler": {k: (getattr(c.sampler, k) if k == "top_k" else f32_bits(getattr(c.sampler, k)))
                        for k in SAMPLER_FIELDS},
            "uniform": f32_bits(c.uniform)}


def result_dict(r):
    return {"source_rank": r.source_rank, "destination_rank": r.destination_rank,
            "token_index": r.token_index, "token": r.token, "logit": f32_bits(r.logit)}


def make_config(src=0, dst=4, flags=0, slot=0, index=17, uniform=0.25, **sampler):
    c = Config(src, dst, flags, slot, index)
    for k, v in sampler.items():
        setattr(c.sampler, k, v)
    c.uniform = uniform
    return c


def main():
    if not LIB.exists():
        sys.exit(f"{LIB} is missing: run `make -C oracle ref` first")
    lib = C.CDLL(str(LIB))
    lib.fg_output_config_encode.argtypes = [C.c_void_p, C.POINTER(Config), C.POINTER(Err)]
    lib.fg_output_config_decode.argtypes = [C.POINTER(Config), C.c_void_p, C.c_uint32, C.POINTER(Err)]
    lib.fg_output_result_encode.argtypes = [C.c_void_p, C.POINTER(Result), C.POINTER(Err)]
    lib.fg_output_result_decode.argtypes = [C.POINTER(Result), C.c_void_p, C.c_uint32, C.POINTER(Err)]
    for f in (lib.fg_output_config_encode, lib.fg_output_config_decode,
              lib.fg_output_result_encode, lib.fg_output_result_decode):
        f.restype = C.c_int
    sampled = dict(temperature=0.7, top_p=0.8, top_k=20, presence_penalty=1.5,
                   frequency_penalty=0.25, repetition_penalty=1.05, min_p=0.0)
    configs = [
        make_config(),                                                 # all controls 0
        make_config(flags=1), make_config(flags=3), make_config(flags=2),
        make_config(slot=1), make_config(slot=2), make_config(src=7), make_config(src=8),
        make_config(dst=5), make_config(dst=0), make_config(index=0xFFFFFFFF),
        make_config(uniform=0.0), make_config(uniform=0.99999994), make_config(uniform=1.0),
        make_config(uniform=-0.0), make_config(uniform=-1e-30), make_config(uniform=math.nan),
        make_config(uniform=math.inf),
        make_config(**sampled), make_config(**dict(sampled, top_k=64)),
        make_config(**dict(sampled, top_k=65)), make_config(**dict(sampled, top_k=0)),
        make_config(**dict(sampled, temperature=0.0, top_k=1)),
        make_config(**dict(sampled, repetition_penalty=0.0)),
        make_config(**dict(sampled, min_p=0.1)), make_config(**dict(sampled, presence_penalty=2.01)),
        make_config(**dict(sampled, top_p=0.0)), make_config(**dict(sampled, top_p=1.0)),
        make_config(top_k=1),                                          # one control nonzero
        make_config(repetition_penalty=1.0),
        make_config(temperature=-0.0),                                 # -0 counts as 0
    ]
    enc = []
    valid_wires = []
    for c in configs:
        buf = (C.c_uint8 * 40)(*([0xAB] * 40))
        e = Err()
        st = lib.fg_output_config_encode(buf, C.byref(c), C.byref(e))
        wire = bytes(buf).hex() if st == 0 else None
        enc.append({"config": config_dict(c), "status": st, "wire": wire})
        if st == 0:
            valid_wires.append(bytes(buf))
    # Decode: every valid wire, then mutations of a few of them.
    payloads = [w for w in valid_wires]
    base = valid_wires[0]
    sampled_wire = [w for w in valid_wires if w[19] == 20][0]
    for b in (base, sampled_wire):
        for i in (0, 1, 2, 3):
            for v in (1, 2, 3, 4, 5, 7, 8, 0x80, 0xFF):
                m = bytearray(b); m[i] = v; payloads.append(bytes(m))
        for i in range(4, 40, 4):
            for word in (0x00000000, 0x3F800000, 0x7FC00000, 0x7F800000, 0xFF800000, 0x00000041,
                         0x3F7FFFFF, 0xBF800000):
                m = bytearray(b); m[i:i + 4] = word.to_bytes(4, "big"); payloads.append(bytes(m))
    dec = []
    for pl in payloads:
        c = Config()
        e = Err()
        buf = (C.c_uint8 * 40).from_buffer_copy(pl)
        st = lib.fg_output_config_decode(C.byref(c), buf, 40, C.byref(e))
        dec.append({"payload": pl.hex(), "bytes": 40, "status": st,
                    "config": config_dict(c) if st == 0 else None})
    for size in (0, 39, 41, 80):
        c = Config(); e = Err()
        pl = (base * 3)[:max(size, 1)]
        buf = (C.c_uint8 * len(pl)).from_buffer_copy(pl)
        st = lib.fg_output_config_decode(C.byref(c), buf, size, C.byref(e))
        dec.append({"payload": pl.hex(), "bytes": size, "status": st, "config": None})
    results = [Result(4, 0, 91, 42, 12.5), Result(4, 7, 0, 248319, -3.0), Result(4, 8, 1, 1, 1.0),
               Result(3, 0, 1, 1, 1.0), Result(4, 0, 1, 248320, 1.0), Result(4, 0, 1, 1, math.nan),
               Result(4, 0, 1, 1, math.inf), Result(4, 0, 0xFFFFFFFF, 0, -0.0),
               Result(0, 0, 1, 1, 1.0)]
    renc, rwires = [], []
    for r in results:
        buf = (C.c_uint8 * 16)(*([0xAB] * 16))
        e = Err()
        st = lib.fg_output_result_encode(buf, C.byref(r), C.byref(e))
        renc.append({"result": result_dict(r), "status": st, "wire": bytes(buf).hex() if st == 0 else None})
        if st == 0:
            rwires.append(bytes(buf))
    rpayloads = list(rwires)
    for i in range(16):
        for v in (1, 4, 8, 0xFF):
            m = bytearray(rwires[0]); m[i] = v; rpayloads.append(bytes(m))
    rdec = []
    for pl in rpayloads:
        r = Result(); e = Err()
        buf = (C.c_uint8 * 16).from_buffer_copy(pl)
        st = lib.fg_output_result_decode(C.byref(r), buf, 16, C.byref(e))
        rdec.append({"payload": pl.hex(), "bytes": 16, "status": st,
                     "result": result_dict(r) if st == 0 else None})
    for size in (0, 15, 17):
        r = Result(); e = Err()
        pl = (rwires[0] * 2)[:max(size, 1)]
        buf = (C.c_uint8 * len(pl)).from_buffer_copy(pl)
        st = lib.fg_output_result_decode(C.byref(r), buf, size, C.byref(e))
        rdec.append({"payload": pl.hex(), "bytes": size, "status": st, "result": None})
    OUT.write_text(json.dumps({"source": "reference src/protocol.c:1160-1166, 1275-1279 "
                               "compiled by oracle/Makefile (target ref)",
                               "config_encode": enc, "config_decode": dec,
                               "result_encode": renc, "result_decode": rdec}, indent=None) + "\n")
    print(f"wrote {OUT}: {len(enc)} + {len(dec)} config, {len(renc)} + {len(rdec)} result vectors")


if __name__ == "__main__":
    main()
