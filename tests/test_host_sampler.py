"""The C17 host sampler (fg_sampler.h in libfg_sampler_hip.so) against the
reference: golden vectors from the reference's compiled sampler, a C test of
the API, and -- where the reference checkout exists -- the reference's own
tests/test_sampler.c linked against this library instead of its own."""
import ctypes as C
import json
import os
import shutil
import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest

import fg_hip

ROOT = Path(__file__).resolve().parent.parent
GOLDEN = json.loads((Path(__file__).parent / "golden" / "ref_sampler_vectors.json").read_text())
LIBDIR = ROOT / "flash-gordon_amd" / "lib"
REF_TEST = Path("/root/reference/tests/test_sampler.c")


def f32(bits):
    return np.array(bits, dtype=np.uint32).view(np.float32)


def fbits(x):
    return struct.unpack("<I", struct.pack("<f", np.float32(x)))[0]


def test_select_matches_reference_vectors():
    lib = fg_hip.lib()
    for c in GOLDEN["select"]:
        s = f32(c["scores_bits"])
        ids = np.array(c["ids"], dtype=np.uint32)
        cfg = fg_hip.make_config(c["t"], c["p"], c["k"])
        tok, logit, err = C.c_uint32(0), C.c_float(0), fg_hip.FgError()
        st = lib.fg_sampler_select(C.byref(cfg), s.ctypes.data, ids.ctypes.data, s.size,
                                   f32([c["u_bits"]])[0], C.byref(tok), C.byref(logit), C.byref(err))
        assert st == c["status"], c
        if st == 0:
            assert tok.value == c["token"] and fbits(logit.value) == c["logit_bits"], c


def test_penalties_match_reference_vectors():
    lib = fg_hip.lib()
    for c in GOLDEN["penalties"]:
        s = f32(c["scores_bits"]).copy()
        counts = np.array(c["counts"], dtype=np.uint32)
        ids = np.arange(s.size, dtype=np.uint32)
        cfg = fg_hip.make_config(1.0, 1.0, 1, c["presence"], c["frequency"], c["repetition"])
        lib.fg_sampler_apply_penalties(s.ctypes.data, ids.ctypes.data, counts.ctypes.data, s.size,
                                       C.byref(cfg))
        assert s.view(np.uint32).tolist() == c["out_bits"]


def test_uniform_streams_match_reference_vectors():
    lib = fg_hip.lib()
    for c in GOLDEN["uniforms"]:
        st = fg_hip.SamplerState()
        lib.fg_sampler_state_init(C.byref(st), int(c["seed"]))
        got = [fbits(lib.fg_sampler_uniform(C.byref(st))) for _ in range(16)]
        assert got == c["uniform_bits"]


def test_validation_matches_reference_vectors():
    lib = fg_hip.lib()
    for c in GOLDEN["validate"]:
        cfg = fg_hip.make_config(c["t"], c["p"], c["k"], c["presence"], c["frequency"],
                                 c["repetition"], c["min_p"])
        err = fg_hip.FgError()
        st = lib.fg_sampler_config_validate(C.byref(cfg), C.byref(err))
        assert st == c["status"] and err.message.decode() == c["message"], c


def _cc():
    return shutil.which("gcc") or shutil.which("cc")


def _run_c_test(src: Path, tmp_path: Path, include: Path):
    exe = tmp_path / src.stem
    subprocess.run([_cc(), "-std=c17", "-D_GNU_SOURCE", "-O2", f"-I{include}", str(src),
                    f"-L{LIBDIR}", "-lfg_sampler_hip", f"-Wl,-rpath,{LIBDIR}", "-lm", "-o", str(exe)],
                   check=True)
    return subprocess.run([str(exe)], capture_output=True, text=True,
                          env=dict(os.environ, LD_LIBRARY_PATH=str(LIBDIR)))


@pytest.mark.skipif(_cc() is None, reason="no C compiler")
def test_c_api_test(tmp_path):
    r = _run_c_test(ROOT / "tests" / "c" / "test_fg_sampler.c", tmp_path, ROOT / "include")
    assert r.returncode == 0, r.stderr


@pytest.mark.skipif(not REF_TEST.exists() or _cc() is None,
                    reason="reference checkout not present (build container only)")
def test_reference_test_sampler_links_against_this_library(tmp_path):
    """Drop-in check: the reference's own unit test, compiled against this
    build's include/fg_sampler.h and linked to libfg_sampler_hip.so."""
    r = _run_c_test(REF_TEST, tmp_path, ROOT / "include")
    assert r.returncode == 0, r.stderr
