"""The C ABI library loads and exports every function include/*.h declares;
argument checks that run before any device work return FG_ERR_ARGUMENT."""
import ctypes as C
import re
from pathlib import Path

import fg_hip

ROOT = Path(__file__).resolve().parent.parent


def declared_functions():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"^\s*(?:[A-Za-z_][\w\s\*]*?)\b(fg_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_every_declared_symbol_is_exported():
    lib = fg_hip.load_library()
    names = declared_functions()
    assert {"fg_sampler_select", "fg_sampler_hip_sample", "fg_hip_topk_select"} <= names
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    assert set(fg_hip.EXPORTS) == names


def test_argument_errors_without_device_work():
    lib = fg_hip.lib()
    err = fg_hip.FgError()
    assert lib.fg_hip_apply_penalties(None, None, 0, 0.0, 0.0, 1.0, None, C.byref(err)) == 2
    assert b"penalty" in err.message
    n = C.c_uint32(0)
    err = fg_hip.FgError()
    assert lib.fg_hip_topk_select(None, None, None, None, 10, 0, C.byref(n), None, C.byref(err)) == 2
    assert err.message == b"invalid generation top-k selection dispatch"
    err = fg_hip.FgError()
    assert lib.fg_hip_argmax_reduce(None, None, None, None, 0, C.byref(n), None, C.byref(err)) == 2
    err = fg_hip.FgError()
    h = C.c_void_p()
    assert lib.fg_sampler_hip_create(C.byref(h), 0, 4, C.byref(err)) == 2
    assert lib.fg_sampler_hip_create(C.byref(h), 0x80000000, 4, C.byref(err)) == 2
    err = fg_hip.FgError()
    assert lib.fg_sampler_hip_sample(None, None, None, C.byref(err)) == 2
    assert lib.fg_sampler_hip_set_configs(None, None, 0, 0, None, C.byref(err)) == 2
    assert lib.fg_hip_history_build(None, 0, 0, None, None, 0, None, None, C.byref(err)) == 2
    assert lib.fg_hip_topk_reduce_all(None, None, None, None, 5, None, C.byref(n), None,
                                      C.byref(err)) == 2
    lib.fg_sampler_hip_destroy(None)


def test_reduce_all_workspace_bytes():
    """Fixed part (header, six 4096-bucket tables, a 6144-entry list, a bound
    and a slot of 8 bytes each for 1,024 tiles), then per 4096-score tile a
    1024-entry region of 12-byte entries."""
    fixed = 64 + 6 * 4096 * 4 + 6144 * 12 + 1024 * 16
    for count, tiles in ((1, 1), (4096, 1), (4097, 2), (262_144, 64), (300_000, 74)):
        assert fg_hip.topk_reduce_all_workspace_bytes(count) == fixed + tiles * 1024 * 12


def test_missing_library_fails_loudly(tmp_path):
    import pytest
    with pytest.raises(RuntimeError, match="not built"):
        fg_hip.load_library(tmp_path / "nope.so")


def test_history_offsets_must_be_64_bit():
    """The history entry points read `const uint64_t *offsets`: the binding
    refuses narrower offsets before any device call."""
    import pytest
    import torch
    off32 = torch.zeros(5, dtype=torch.int32)
    with pytest.raises(ValueError):
        fg_hip.history_build_wire(None, 8, 8, None, off32, 4, None)
    with pytest.raises(ValueError):
        fg_hip.history_build(None, 8, 8, None, off32, 4, None)
    with pytest.raises(ValueError):
        fg_hip.history_build(None, 8, 8, None, torch.zeros(4, dtype=torch.int64), 4, None)
