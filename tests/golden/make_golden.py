"""Writes tests/golden/ref_sampler_vectors.json from the reference's own host
sampler, compiled from its sources by `make -C oracle ref` into
oracle/_ref/libfg_ref_sampler.so (reference src/sampler.c, src/util.c).

The vectors pin, on fixed inputs, what the reference computes:
  * fg_sampler_select (src/sampler.c:80-122): status, token id and logit bits,
    including ties, non-finite candidates, uniforms at and past the ends, and
    near-boundary top-p / draw cases;
  * fg_sampler_apply_penalties (src/sampler.c:46-60): output bits;
  * fg_sampler_uniform / state_init (src/sampler.c:62-73): the first uniforms
    of several seeds, as bits;
  * fg_sampler_config_validate (src/sampler.c:24-38): status per config.
Run in the build container (where /root/reference exists):
    python tests/golden/make_golden.py
"""
from __future__ import annotations

import ctypes as C
import json
import struct
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "oracle"))
import oracle_ffi as O  # noqa: E402

OUT = Path(__file__).resolve().parent / "ref_sampler_vectors.json"


def fbits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", np.float32(x)))[0]


def cfg(t, p, k, pres=0.0, freq=0.0, rep=1.0, min_p=0.0, seed=0):
    return O.RefConfig(t, p, k, pres, freq, rep, min_p, seed)


def select_cases(rng):
    cases = []
    # Known answers of the reference's own test (tests/test_sampler.c:31-46).
    base = dict(scores=[5.0, 4.0, 3.0], ids=[9, 3, 1])
    for t, p, k, u in [(1.0, 1.0, 2, 0.3), (1.0, 1.0, 3, 0.8), (0.1, 1.0, 3, 0.8),
                       (0.1, 0.5, 3, 0.99), (0.01, 1.0, 3, 0.99)]:
        cases.append(dict(base, t=t, p=p, k=k, u=u))
    cases.append(dict(scores=[1.0, 1.0], ids=[8, 2], t=0.0, p=1.0, k=1, u=0.5))
    # Random sets: sizes 1..64, temperatures, top-p, top-k, uniforms.
    for _ in range(400):
        n = int(rng.integers(1, 65))
        kind = rng.integers(0, 4)
        if kind == 0:
            s = rng.normal(0, 3, n)
        elif kind == 1:
            s = np.round(rng.normal(0, 2, n) * 2) / 2          # ties
        elif kind == 2:
            s = rng.normal(0, 0.05, n)                           # flat
        else:
            s = rng.normal(0, 3, n)
            s[rng.integers(0, n, max(1, n // 8))] = rng.choice([np.nan, np.inf, -np.inf])
        ids = rng.choice(200_000, n, replace=False)
        t = float(rng.choice([0.0, 0.3, 0.7, 1.0, 1.5]))
        p = float(rng.choice([0.1, 0.5, 0.8, 0.9, 0.95, 1.0]))
        k = int(rng.integers(1, 65))
        u = float(rng.choice([rng.random(), 0.0, 0.999999, 1.0, -0.5, np.nan]))
        cases.append(dict(scores=s.astype(np.float32).tolist(), ids=ids.tolist(), t=t, p=p, k=k, u=u))
    return cases


def run_select(ref, c):
    n = len(c["scores"])
    s = np.array(c["scores"], dtype=np.float32)
    ids = np.array(c["ids"], dtype=np.uint32)
    tok, logit = C.c_uint32(0xFFFFFFFF), C.c_float(0.0)
    err = O.RefError()
    st = ref.fg_sampler_select(C.byref(cfg(c["t"], c["p"], c["k"])), s.ctypes.data_as(C.c_void_p),
                               ids.ctypes.data_as(C.c_void_p), n, np.float32(c["u"]),
                               C.byref(tok), C.byref(logit), C.byref(err))
    return dict(status=int(st), token=int(tok.value) if st == 0 else None,
                logit_bits=fbits(logit.value) if st == 0 else None)


def main():
    if not O.reference_available():
        sys.exit("oracle/_ref/libfg_ref_sampler.so is missing: run `make -C oracle ref` first")
    ref = O.reference()
    rng = np.random.default_rng(20261201)

    sel = []
    for c in select_cases(rng):
        out = run_select(ref, c)
        c = dict(c, scores_bits=[fbits(x) for x in c["scores"]])
        del c["scores"]
        c["u_bits"] = fbits(c.pop("u"))
        sel.append(dict(c, **out))

    pen = []
    for i in range(60):
        n = int(rng.integers(1, 300))
        s = rng.normal(0, 4, n).astype(np.float32)
        if i % 5 == 0:
            s[: min(n, 3)] = np.array([0.0, -0.0, np.nan], dtype=np.float32)[: min(n, 3)]
        counts = np.zeros(n, dtype=np.uint32)
        hot = rng.integers(0, n, max(1, n // 3))
        counts[hot] = rng.integers(1, 5000, hot.size).astype(np.uint32)
        if i % 7 == 0:
            counts[0] = 0xFFFFFFFF
        pres = float(np.float32(rng.uniform(-2, 2)))
        freq = float(np.float32(rng.uniform(-2, 2)))
        rep = float(np.float32(rng.choice([1.0, 1.05, 1.1, 2.0, 0.7])))
        ids = np.arange(n, dtype=np.uint32)
        out = s.copy()
        ref.fg_sampler_apply_penalties(out.ctypes.data_as(C.c_void_p), ids.ctypes.data_as(C.c_void_p),
                                       counts.ctypes.data_as(C.c_void_p), n,
                                       C.byref(cfg(1.0, 1.0, 1, pres, freq, rep)))
        pen.append(dict(scores_bits=s.view(np.uint32).tolist(), counts=counts.tolist(),
                        presence=pres, frequency=freq, repetition=rep,
                        out_bits=out.view(np.uint32).tolist()))

    uni = []
    for seed in [0, 1, 42, 0x9E3779B97F4A7C15, 2**64 - 1, 123456789]:
        state = C.c_uint64(0)
        ref.fg_sampler_state_init(C.byref(state), seed)
        vals = [fbits(ref.fg_sampler_uniform(C.byref(state))) for _ in range(16)]
        uni.append(dict(seed=str(seed), uniform_bits=vals))

    val = []
    for t, p, k, pres, freq, rep, min_p in [
            (1.0, 0.95, 20, 0, 0, 1, 0), (1.0, 0.95, 20, 2.0, -2.0, 1, 0),
            (1.0, 0.95, 20, 2.01, 0, 1, 0), (1.0, 0.95, 20, -2.01, 0, 1, 0),
            (1.0, 0.95, 20, 0, 2.01, 1, 0), (1.0, 0.95, 20, 0, -2.01, 1, 0),
            (1.0, 0.95, 20, 0, 0, 0.0, 0), (1.0, 0.95, 20, 0, 0, 1, 0.1),
            (0.7, 0.8, 20, 1.5, 0, 1, 0), (1.0, 0.95, 65, 0, 0, 1, 0), (1.0, 0.95, 0, 0, 0, 1, 0),
            (-0.1, 0.95, 20, 0, 0, 1, 0), (1.0, 0.0, 20, 0, 0, 1, 0), (1.0, 1.0, 64, 0, 0, 1, 0),
            (float("inf"), 0.9, 20, 0, 0, 1, 0), (1.0, float("nan"), 20, 0, 0, 1, 0),
            (1.0, 0.9, 20, 0, 0, -1.0, 0), (0.0, 1.0, 1, 0, 0, 1, 0)]:
        err = O.RefError()
        st = ref.fg_sampler_config_validate(C.byref(cfg(t, p, k, pres, freq, rep, min_p)), C.byref(err))
        val.append(dict(t=t, p=p, k=k, presence=pres, frequency=freq, repetition=rep, min_p=min_p,
                        status=int(st), message=err.message.decode()))

    doc = dict(source="reference src/sampler.c + src/util.c compiled by oracle/Makefile (ref)",
               select=sel, penalties=pen, uniforms=uni, validate=val)
    OUT.write_text(json.dumps(doc, separators=(",", ":")))
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes): {len(sel)} select, {len(pen)} penalty, "
          f"{len(uni)} uniform streams, {len(val)} validations")


if __name__ == "__main__":
    main()
