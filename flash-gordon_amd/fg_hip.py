"""ctypes binding of lib/libfg_sampler_hip.so (include/fg_sampler.h and
include/fg_sampler_hip.h).

This is the Python face of the C ABI, used by the tests, smoke() and bench.py.
Device buffers are passed as torch tensors (their data_ptr()); torch only
provides device memory and streams.  Every call goes to the HIP library; there
is no fallback, and a missing library raises at load time.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "lib" / "libfg_sampler_hip.so"

FG_OK = 0
FG_ERR_ARGUMENT = 2
FG_ERR_IO = 3
FG_ERR_FORMAT = 4
FG_ERR_MISMATCH = 5
FG_ERR_OOM = 6
FG_ERR_UNAVAILABLE = 7
FG_ERR_LIMIT = 8
FG_ERR_INTERRUPTED = 9

INVALID_ID = 0xFFFFFFFF
MAX_TOPK = 64
ALLOW_FULL_VOCAB = 1

# Every symbol include/*.h declares (checked by tests/test_abi.py).
EXPORTS = (
    "fg_error_set",
    "fg_sampler_config_greedy", "fg_sampler_config_defaults", "fg_sampler_config_validate",
    "fg_sampler_state_init", "fg_sampler_uniform", "fg_sampler_select",
    "fg_sampler_penalties_active", "fg_sampler_apply_penalties",
    "fg_hip_apply_penalties", "fg_hip_argmax_reduce", "fg_hip_topk_select", "fg_hip_topk_reduce",
    "fg_hip_topk_reduce_all", "fg_hip_topk_reduce_all_workspace_bytes",
    "fg_hip_history_build", "fg_hip_history_build_wire",
    "fg_output_history_encode", "fg_output_history_encode_vocab",
    "fg_output_history_decode", "fg_output_history_decode_vocab",
    "fg_sampler_hip_create", "fg_sampler_hip_destroy", "fg_sampler_hip_set_configs",
    "fg_sampler_hip_sample", "fg_sampler_hip_history_increment", "fg_sampler_hip_sample_static",
    "fg_sampler_hip_set_wait_limit",
    "fg_output_better", "fg_output_combine", "fg_output_split_way_for_rank",
    "fg_output_split_rank", "fg_output_split_span", "fg_output_split_combine_finalists",
    "fg_hip_output_slice_create", "fg_hip_output_slice_destroy", "fg_hip_output_slice_ways",
    "fg_hip_output_slice_reduce", "fg_hip_output_split_combine",
    "fg_hip_output_slice_reduce_combine", "fg_hip_output_slice_set_wait_limit",
    "fg_f16_to_f32", "fg_f32_to_f16", "fg_quantize_q8_0", "fg_dequantize_q8_0",
    "fg_q8_0_cooked_tile_bytes", "fg_q8_0_cooked_matrix_bytes", "fg_cook_q8_0_rows",
    "fg_uncook_q8_0_rows", "fg_hip_dense_q8_0_cooked", "fg_hip_output_slice_run_dense",
    "fg_hip_output_slice_run_dense_sampled",
    "fg_sampler_hip_plan", "fg_sampler_hip_block",
    "fg_output_config_encode", "fg_output_config_decode", "fg_output_result_encode",
    "fg_output_result_decode", "fg_output_configs_batch", "fg_output_results_encode_batch",
)

ROWS_NUCLEUS = 1
ROWS_UNLIKE_COST = 2


class FgError(C.Structure):
    _fields_ = [("code", C.c_int), ("message", C.c_char * 512)]


class Geometry(C.Structure):
    """fg_sampler_hip_geometry (include/fg_sampler_hip.h)."""
    _fields_ = [("chunks", C.c_uint32), ("split", C.c_uint32), ("wave_elems", C.c_uint32),
                ("wave_elems_b", C.c_uint32), ("pace", C.c_uint32)]


class SamplerConfig(C.Structure):
    """fg_sampler_config (include/fg_sampler.h)."""
    _fields_ = [
        ("temperature", C.c_float), ("top_p", C.c_float), ("top_k", C.c_uint32),
        ("presence_penalty", C.c_float), ("frequency_penalty", C.c_float),
        ("repetition_penalty", C.c_float), ("min_p", C.c_float), ("seed", C.c_uint64),
    ]


class SamplerState(C.Structure):
    _fields_ = [("state", C.c_uint64)]


class OutputConfig(C.Structure):
    """fg_output_config (include/fg_output_wire.h)."""
    _fields_ = [("source_rank", C.c_uint8), ("destination_rank", C.c_uint8),
                ("flags", C.c_uint8), ("session_slot", C.c_uint8), ("token_index", C.c_uint32),
                ("sampler", SamplerConfig), ("uniform", C.c_float)]


class OutputResult(C.Structure):
    """fg_output_result (include/fg_output_wire.h)."""
    _fields_ = [("source_rank", C.c_uint8), ("destination_rank", C.c_uint8),
                ("token_index", C.c_uint32), ("token", C.c_uint32), ("logit", C.c_float)]


class Batch(C.Structure):
    """fg_sampler_hip_batch (include/fg_sampler_hip.h)."""
    _fields_ = [
        ("logits", C.c_void_p), ("logits_stride", C.c_uint64),
        ("counts", C.c_void_p), ("counts_stride", C.c_uint64),
        ("uniforms", C.c_void_p), ("rows", C.c_uint32),
        ("tokens", C.c_void_p), ("token_logits", C.c_void_p), ("row_status", C.c_void_p),
        ("penalised", C.c_void_p), ("logprobs", C.c_uint32),
        ("logprob_values", C.c_void_p), ("logprob_ids", C.c_void_p),
    ]


class OutputHistory(C.Structure):
    """fg_output_history (include/fg_history.h)."""
    _fields_ = [("tokens", C.c_void_p), ("count", C.c_uint32), ("session_slot", C.c_uint8)]


HISTORY_HEADER_BYTES = 8
HISTORY_Q38_VOCAB = 248320


class FgStatusError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"fg_status {code}: {message}")
        self.code = code
        self.message = message


def load_library(path: Path | str | None = None) -> C.CDLL:
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise RuntimeError(
            f"HIP sampling library not built: {p} is missing (run __graft_entry__.build())")
    lib = C.CDLL(str(p))
    P = C.c_void_p
    E = C.POINTER(FgError)
    u32, u64, f32 = C.c_uint32, C.c_uint64, C.c_float
    sig = {
        "fg_sampler_config_greedy": (None, [C.POINTER(SamplerConfig)]),
        "fg_sampler_config_defaults": (None, [C.POINTER(SamplerConfig)]),
        "fg_sampler_config_validate": (C.c_int, [C.POINTER(SamplerConfig), E]),
        "fg_sampler_state_init": (None, [C.POINTER(SamplerState), u64]),
        "fg_sampler_uniform": (f32, [C.POINTER(SamplerState)]),
        "fg_sampler_select": (C.c_int, [C.POINTER(SamplerConfig), P, P, u32, f32, P, P, E]),
        "fg_sampler_penalties_active": (C.c_bool, [C.POINTER(SamplerConfig)]),
        "fg_sampler_apply_penalties": (None, [P, P, P, u32, C.POINTER(SamplerConfig)]),
        "fg_hip_apply_penalties": (C.c_int, [P, P, u32, f32, f32, f32, P, E]),
        "fg_hip_argmax_reduce": (C.c_int, [P, P, P, P, u32, C.POINTER(u32), P, E]),
        "fg_hip_topk_select": (C.c_int, [P, P, P, P, u32, u32, C.POINTER(u32), P, E]),
        "fg_hip_topk_reduce": (C.c_int, [P, P, P, P, u32, C.POINTER(u32), P, E]),
        "fg_hip_topk_reduce_all": (C.c_int, [P, P, P, P, u32, P, C.POINTER(u32), P, E]),
        "fg_hip_topk_reduce_all_workspace_bytes": (u64, [u32]),
        "fg_hip_history_build": (C.c_int, [P, u64, u32, P, P, u32, P, P, E]),
        "fg_hip_history_build_wire": (C.c_int, [P, u64, u32, P, P, u32, P, P, P, E]),
        "fg_output_history_encode": (C.c_int, [P, u32, C.POINTER(u32), C.POINTER(OutputHistory), E]),
        "fg_output_history_encode_vocab":
            (C.c_int, [P, u32, C.POINTER(u32), C.POINTER(OutputHistory), u32, E]),
        "fg_output_history_decode": (C.c_int, [C.POINTER(OutputHistory), P, u32, P, u32, E]),
        "fg_output_history_decode_vocab":
            (C.c_int, [C.POINTER(OutputHistory), P, u32, P, u32, u32, E]),
        "fg_sampler_hip_create": (C.c_int, [C.POINTER(P), u32, u32, E]),
        "fg_sampler_hip_destroy": (None, [P]),
        "fg_sampler_hip_set_configs": (C.c_int, [P, C.POINTER(SamplerConfig), u32, u32, P, E]),
        "fg_sampler_hip_sample": (C.c_int, [P, C.POINTER(Batch), P, E]),
        "fg_sampler_hip_sample_static":
            (C.c_int, [u32, C.POINTER(SamplerConfig), u32, C.POINTER(Batch), P, E]),
        "fg_sampler_hip_history_increment": (C.c_int, [P, P, u64, P, P, u32, P, E]),
        "fg_sampler_hip_set_wait_limit": (C.c_int, [P, u64, E]),
        "fg_output_better": (C.c_bool, [f32, u32, f32, u32]),
        "fg_output_combine": (None, [f32, u32, f32, u32, C.POINTER(f32), C.POINTER(u32)]),
        "fg_output_split_way_for_rank": (C.c_bool, [u32, u32, C.POINTER(u32)]),
        "fg_output_split_rank": (u32, [u32, u32]),
        "fg_output_split_span": (None, [u32, u32, C.POINTER(u32), C.POINTER(u32)]),
        "fg_output_split_combine_finalists":
            (C.c_int, [u32, f32, u32, P, P, P, u32, C.POINTER(u32), C.POINTER(f32), E]),
        "fg_hip_output_slice_create": (C.c_int, [C.POINTER(P), u32, u32, u32, u32, u32, E]),
        "fg_hip_output_slice_destroy": (None, [P]),
        "fg_hip_output_slice_ways": (u32, [P]),
        "fg_hip_output_slice_reduce": (C.c_int, [P, P, u64, u32, P, P, P, P, E]),
        "fg_hip_output_slice_reduce_combine":
            (C.c_int, [P, P, u64, u32, P, P, P, P, P, P, P, P, P, E]),
        "fg_hip_output_slice_set_wait_limit": (C.c_int, [P, u64, E]),
        "fg_hip_output_split_combine":
            (C.c_int, [P, P, P, P, P, P, u32, u32, u32, P, P, P, E]),
        "fg_f16_to_f32": (f32, [C.c_uint16]),
        "fg_f32_to_f16": (C.c_uint16, [f32]),
        "fg_quantize_q8_0": (None, [P, P, u64]),
        "fg_dequantize_q8_0": (None, [P, P, u64]),
        "fg_q8_0_cooked_tile_bytes": (u64, [u32]),
        "fg_q8_0_cooked_matrix_bytes": (u64, [u32, u32]),
        "fg_cook_q8_0_rows": (C.c_bool, [P, P, u64, u32, u32]),
        "fg_uncook_q8_0_rows": (C.c_bool, [P, P, u64, u32, u32]),
        "fg_hip_dense_q8_0_cooked": (C.c_int, [P, P, P, u32, u32, u32, f32, P, E]),
        "fg_hip_output_slice_run_dense_sampled":
            (C.c_int, [P, P, P, u32, u32, f32, C.POINTER(SamplerConfig), P, u64, P, P, P, P, P, E]),
        "fg_hip_output_slice_run_dense":
            (C.c_int, [P, P, P, u32, u32, f32, P, P, P, P, P, E]),
        "fg_sampler_hip_plan": (C.c_int, [u32, u32, u32, C.POINTER(Geometry), E]),
        "fg_output_config_encode": (C.c_int, [P, C.POINTER(OutputConfig), E]),
        "fg_output_config_decode": (C.c_int, [C.POINTER(OutputConfig), P, u32, E]),
        "fg_output_result_encode": (C.c_int, [P, C.POINTER(OutputResult), E]),
        "fg_output_result_decode": (C.c_int, [C.POINTER(OutputResult), P, u32, E]),
        "fg_output_configs_batch": (C.c_int, [P, u32, P, P, E]),
        "fg_output_results_encode_batch": (C.c_int, [P, P, P, P, P, u32, C.POINTER(u32), E]),
        "fg_sampler_hip_block": (C.c_int, [C.POINTER(Geometry), u32, u32, u32, u32,
                                           C.POINTER(u32), C.POINTER(u32), C.POINTER(u32),
                                           C.POINTER(u32), E]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_LIB: C.CDLL | None = None


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        _LIB = load_library()
    return _LIB


def _check(status: int, err: FgError) -> None:
    if status != FG_OK:
        raise FgStatusError(status, err.message.decode(errors="replace"))


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(stream) -> int | None:
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    return int(stream)


def make_config(temperature=1.0, top_p=0.95, top_k=20, presence=0.0, frequency=0.0,
                repetition=1.0, min_p=0.0, seed=0x9E3779B97F4A7C15) -> SamplerConfig:
    return SamplerConfig(temperature, top_p, top_k, presence, frequency, repetition, min_p, seed)


# ---- unit kernels ----------------------------------------------------------

def apply_penalties(logits, counts, presence, frequency, repetition, stream=None):
    err = FgError()
    _check(lib().fg_hip_apply_penalties(_ptr(logits), _ptr(counts), logits.numel(),
                                        presence, frequency, repetition, _stream(stream),
                                        C.byref(err)), err)


def argmax_reduce(out_scores, out_ids, in_scores, in_ids, count, stream=None) -> int:
    err = FgError()
    n = C.c_uint32(0)
    _check(lib().fg_hip_argmax_reduce(_ptr(out_scores), _ptr(out_ids), _ptr(in_scores),
                                      _ptr(in_ids), count, C.byref(n), _stream(stream),
                                      C.byref(err)), err)
    return n.value


def topk_select(out_scores, out_ids, in_scores, in_ids, count, k, stream=None) -> int:
    err = FgError()
    n = C.c_uint32(0)
    _check(lib().fg_hip_topk_select(_ptr(out_scores), _ptr(out_ids), _ptr(in_scores),
                                    _ptr(in_ids), count, k, C.byref(n), _stream(stream),
                                    C.byref(err)), err)
    return n.value


def topk_reduce(out_scores, out_ids, in_scores, in_ids, count, stream=None) -> int:
    """fg_hip_topk_reduce: sorted top-512 per 4096-value tile; returns the output count."""
    err = FgError()
    n = C.c_uint32(0)
    _check(lib().fg_hip_topk_reduce(_ptr(out_scores), _ptr(out_ids), _ptr(in_scores),
                                    _ptr(in_ids), count, C.byref(n), _stream(stream),
                                    C.byref(err)), err)
    return n.value


def topk_reduce_all_workspace_bytes(count) -> int:
    """fg_hip_topk_reduce_all_workspace_bytes: the workspace for `count` scores."""
    return int(lib().fg_hip_topk_reduce_all_workspace_bytes(count))


def topk_reduce_all(out_scores, out_ids, in_scores, in_ids, count, workspace,
                    stream=None) -> int:
    """fg_hip_topk_reduce_all: the whole top-512 scan in one launch; returns the output count."""
    err = FgError()
    n = C.c_uint32(0)
    _check(lib().fg_hip_topk_reduce_all(_ptr(out_scores), _ptr(out_ids), _ptr(in_scores),
                                        _ptr(in_ids), count, _ptr(workspace), C.byref(n),
                                        _stream(stream), C.byref(err)), err)
    return n.value


def _check_u64_offsets(offsets, rows):
    """The history entry points take `const uint64_t *offsets` (rows + 1)."""
    size = getattr(offsets, "element_size", None)
    if size is not None and (size() != 8 or offsets.numel() < rows + 1):
        raise ValueError("offsets must hold rows + 1 64-bit entries")


def history_build(counts, stride, vocab, ids, offsets, rows, row_status, stream=None):
    """fg_hip_history_build: count tables from id lists; per-row status on the device."""
    _check_u64_offsets(offsets, rows)
    err = FgError()
    _check(lib().fg_hip_history_build(_ptr(counts), stride, vocab, _ptr(ids), _ptr(offsets),
                                      rows, _ptr(row_status), _stream(stream), C.byref(err)), err)


def history_build_wire(counts, stride, vocab, payloads, offsets, rows, row_status,
                       row_slot=None, stream=None):
    """fg_hip_history_build_wire: count tables from FG_MSG_OUTPUT_HISTORY payloads."""
    _check_u64_offsets(offsets, rows)
    err = FgError()
    _check(lib().fg_hip_history_build_wire(_ptr(counts), stride, vocab, _ptr(payloads),
                                           _ptr(offsets), rows, _ptr(row_status),
                                           _ptr(row_slot), _stream(stream), C.byref(err)), err)


def history_encode(tokens, session_slot=0, vocab=None, capacity=None):
    """fg_output_history_encode(_vocab): the payload bytes; raises FgStatusError."""
    import numpy as np
    t = np.ascontiguousarray(tokens, dtype=np.uint32)
    h = OutputHistory(t.ctypes.data if t.size else None, t.size, session_slot)
    cap = capacity if capacity is not None else HISTORY_HEADER_BYTES + 4 * t.size
    buf = (C.c_uint8 * max(cap, 1))()
    n = C.c_uint32(0)
    err = FgError()
    if vocab is None:
        st = lib().fg_output_history_encode(buf, cap, C.byref(n), C.byref(h), C.byref(err))
    else:
        st = lib().fg_output_history_encode_vocab(buf, cap, C.byref(n), C.byref(h), vocab,
                                                  C.byref(err))
    _check(st, err)
    return bytes(buf[:n.value])


def history_decode(payload: bytes, capacity: int, vocab=None):
    """fg_output_history_decode(_vocab): (tokens as a list, session_slot)."""
    import numpy as np
    storage = np.zeros(max(capacity, 1), dtype=np.uint32)
    h = OutputHistory()
    src = (C.c_uint8 * max(len(payload), 1)).from_buffer_copy(payload or b"\0")
    err = FgError()
    sp = storage.ctypes.data if capacity else None
    if vocab is None:
        st = lib().fg_output_history_decode(C.byref(h), sp, capacity, src, len(payload),
                                            C.byref(err))
    else:
        st = lib().fg_output_history_decode_vocab(C.byref(h), sp, capacity, src, len(payload),
                                                  vocab, C.byref(err))
    _check(st, err)
    return storage[:h.count].tolist(), h.session_slot


# ---- Q8_0 weights (host) and products (device) -----------------------------

def quantize_q8_0(x):
    """fg_quantize_q8_0 over a float32 array (size a multiple of 32) -> bytes as uint8."""
    import numpy as np
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.zeros(x.size // 32 * 34, dtype=np.uint8)
    lib().fg_quantize_q8_0(x.ctypes.data, out.ctypes.data, x.size)
    return out


def cook_q8_0(packed, width, rows):
    """fg_cook_q8_0_rows: packed Q8_0 rows -> cooked tiles (uint8 array)."""
    import numpy as np
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    n = lib().fg_q8_0_cooked_matrix_bytes(width, rows)
    out = np.empty(n, dtype=np.uint8)
    if not n or not lib().fg_cook_q8_0_rows(packed.ctypes.data, out.ctypes.data, n, width, rows):
        raise ValueError("fg_cook_q8_0_rows failed")
    return out


def dense_q8_0_cooked(out, weights, x, width, rows, tokens, scale=1.0, stream=None):
    """fg_hip_dense_q8_0_cooked: out[t*rows + r] = scale * W[r] . x[t]."""
    err = FgError()
    _check(lib().fg_hip_dense_q8_0_cooked(_ptr(out), _ptr(weights), _ptr(x), width, rows, tokens,
                                          scale, _stream(stream), C.byref(err)), err)


# ---- vocabulary-split greedy output ----------------------------------------

def split_span(ways: int, way: int) -> tuple[int, int]:
    """fg_output_split_span: (first_row, rows)."""
    first, rows = C.c_uint32(0), C.c_uint32(0)
    lib().fg_output_split_span(ways, way, C.byref(first), C.byref(rows))
    return first.value, rows.value


def split_combine(tokens, logits_out, row_status, part_values, part_ids, part_ranks, rows,
                  ways, vocab, spans, stream=None):
    """fg_hip_output_split_combine; spans = [(first, rows)] by way."""
    first = (C.c_uint32 * len(spans))(*[f for f, _ in spans])
    count = (C.c_uint32 * len(spans))(*[r for _, r in spans])
    err = FgError()
    _check(lib().fg_hip_output_split_combine(
        _ptr(tokens), _ptr(logits_out), _ptr(row_status), _ptr(part_values), _ptr(part_ids),
        _ptr(part_ranks), rows, ways, vocab, first, count, _stream(stream), C.byref(err)), err)


class OutputSlice:
    """Owns an fg_hip_output_slice (vocabulary rows [first_row, first_row + rows))."""

    def __init__(self, vocab, ways, first_row, rows, max_batch_rows):
        self._lib = lib()
        err = FgError()
        h = C.c_void_p()
        _check(self._lib.fg_hip_output_slice_create(C.byref(h), vocab, ways, first_row, rows,
                                                    max_batch_rows, C.byref(err)), err)
        self.handle, self.first_row, self.rows = h, first_row, rows

    def close(self):
        if self.handle:
            self._lib.fg_hip_output_slice_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def ways(self) -> int:
        return self._lib.fg_hip_output_slice_ways(self.handle)

    def run_dense(self, weights, hidden, width, tokens, values, ids, row_status, scale=1.0,
                  logits=None, stream=None):
        """fg_hip_output_slice_run_dense: the slice's cooked rows times hidden,
        fused with each token's finalist."""
        err = FgError()
        _check(self._lib.fg_hip_output_slice_run_dense(
            self.handle, _ptr(weights), _ptr(hidden), width, tokens, scale, _ptr(values),
            _ptr(ids), _ptr(row_status), _ptr(logits), _stream(stream), C.byref(err)), err)

    def run_dense_sampled(self, weights, hidden, width, tokens, configs, uniforms, out_tokens,
                          out_logits, row_status, counts=None, counts_stride=None, scale=1.0,
                          stream=None):
        """fg_hip_output_slice_run_dense_sampled: the LM head fused with
        penalties, the top-k ladder and the select (or the greedy argmax)
        for each token; no logits are written."""
        if len(configs) < tokens:
            raise ValueError(f"{len(configs)} configs for {tokens} tokens")
        arr = (SamplerConfig * len(configs))(*configs)
        stride = counts_stride if counts_stride is not None else (
            counts.stride(0) if counts is not None else 0)
        err = FgError()
        _check(self._lib.fg_hip_output_slice_run_dense_sampled(
            self.handle, _ptr(weights), _ptr(hidden), width, tokens, scale, arr, _ptr(counts),
            stride, _ptr(uniforms), _ptr(out_tokens), _ptr(out_logits), _ptr(row_status),
            _stream(stream), C.byref(err)), err)

    def reduce(self, logits, values, ids, row_status, batch_rows=None, stride=None, stream=None):
        batch_rows = batch_rows if batch_rows is not None else logits.shape[0]
        stride = stride if stride is not None else logits.stride(0)
        err = FgError()
        _check(self._lib.fg_hip_output_slice_reduce(
            self.handle, _ptr(logits), stride, batch_rows, _ptr(values), _ptr(ids),
            _ptr(row_status), _stream(stream), C.byref(err)), err)

    def reduce_combine(self, logits, part_values, part_ids, part_ranks, spans, tokens,
                       logits_out, row_status, batch_rows=None, stride=None, stream=None):
        """fg_hip_output_slice_reduce_combine: the owner's step in one launch;
        spans = [(first, rows)] by way."""
        batch_rows = batch_rows if batch_rows is not None else logits.shape[0]
        stride = stride if stride is not None else logits.stride(0)
        first = (C.c_uint32 * len(spans))(*[f for f, _ in spans])
        count = (C.c_uint32 * len(spans))(*[r for _, r in spans])
        err = FgError()
        _check(self._lib.fg_hip_output_slice_reduce_combine(
            self.handle, _ptr(logits), stride, batch_rows, _ptr(part_values), _ptr(part_ids),
            _ptr(part_ranks), first, count, _ptr(tokens), _ptr(logits_out), _ptr(row_status),
            _stream(stream), C.byref(err)), err)

    def set_wait_limit(self, wait_us):
        """fg_hip_output_slice_set_wait_limit."""
        err = FgError()
        _check(self._lib.fg_hip_output_slice_set_wait_limit(self.handle, wait_us, C.byref(err)),
               err)


# ---- batched sampler -------------------------------------------------------

class HipSampler:
    """Owns an fg_sampler_hip context (device workspace for max_rows rows)."""

    def __init__(self, vocab: int, max_rows: int):
        self._lib = lib()
        err = FgError()
        h = C.c_void_p()
        _check(self._lib.fg_sampler_hip_create(C.byref(h), vocab, max_rows, C.byref(err)), err)
        self.handle = h
        self.vocab = vocab
        self.max_rows = max_rows

    def close(self):
        if self.handle:
            self._lib.fg_sampler_hip_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_configs(self, configs, flags=0, stream=None):
        arr = (SamplerConfig * len(configs))(*configs)
        err = FgError()
        _check(self._lib.fg_sampler_hip_set_configs(self.handle, arr, len(configs), flags,
                                                    _stream(stream), C.byref(err)), err)

    def sample(self, logits, uniforms, tokens, counts=None, token_logits=None, row_status=None,
               penalised=None, logprobs=0, logprob_values=None, logprob_ids=None, rows=None,
               logits_stride=None, counts_stride=None, stream=None):
        rows = rows if rows is not None else logits.shape[0]
        b = Batch(
            _ptr(logits), logits_stride if logits_stride is not None else logits.stride(0),
            _ptr(counts), (counts_stride if counts_stride is not None
                           else (counts.stride(0) if counts is not None else 0)),
            _ptr(uniforms), rows, _ptr(tokens), _ptr(token_logits), _ptr(row_status),
            _ptr(penalised), logprobs, _ptr(logprob_values), _ptr(logprob_ids))
        err = FgError()
        _check(self._lib.fg_sampler_hip_sample(self.handle, C.byref(b), _stream(stream),
                                               C.byref(err)), err)

    def prepare(self, logits, uniforms, tokens, counts=None, token_logits=None, row_status=None,
                penalised=None, logprobs=0, logprob_values=None, logprob_ids=None, rows=None,
                logits_stride=None, counts_stride=None):
        """The batch of a later sample() call marshalled once: returns a
        function of the stream that launches it (for loops over fixed
        buffers, where the per-call argument marshalling would dominate the
        host's part)."""
        rows = rows if rows is not None else logits.shape[0]
        b = Batch(
            _ptr(logits), logits_stride if logits_stride is not None else logits.stride(0),
            _ptr(counts), (counts_stride if counts_stride is not None
                           else (counts.stride(0) if counts is not None else 0)),
            _ptr(uniforms), rows, _ptr(tokens), _ptr(token_logits), _ptr(row_status),
            _ptr(penalised), logprobs, _ptr(logprob_values), _ptr(logprob_ids))
        err = FgError()
        bref, eref, fn, h = C.byref(b), C.byref(err), self._lib.fg_sampler_hip_sample, self.handle

        def launch(stream=None):
            status = fn(h, bref, _stream(stream), eref)
            if status:
                _check(status, err)

        launch.keep = (b, err, logits, uniforms, tokens, counts, token_logits, row_status,
                       penalised, logprob_values, logprob_ids)
        return launch

    def set_wait_limit(self, wait_us: int):
        """The finisher hand-off's wait limit for later calls (microseconds)."""
        err = FgError()
        _check(self._lib.fg_sampler_hip_set_wait_limit(self.handle, wait_us, C.byref(err)), err)

    def history_increment(self, counts, tokens, row_status=None, rows=None, stream=None):
        rows = rows if rows is not None else tokens.numel()
        err = FgError()
        _check(self._lib.fg_sampler_hip_history_increment(
            self.handle, _ptr(counts), counts.stride(0), _ptr(tokens), _ptr(row_status), rows,
            _stream(stream), C.byref(err)), err)


STATIC_MAX_ROWS = 256


def sample_static(vocab, configs, logits, uniforms, tokens, counts=None, token_logits=None,
                  row_status=None, penalised=None, logprobs=0, logprob_values=None,
                  logprob_ids=None, flags=0, rows=None, logits_stride=None, counts_stride=None,
                  stream=None):
    """fg_sampler_hip_sample_static: configs + sample in one call, no sampler
    object, workspace in the library's static device array (allocates
    nothing)."""
    rows = rows if rows is not None else logits.shape[0]
    if len(configs) < rows:
        raise ValueError(f"{len(configs)} configs for {rows} rows")
    arr = (SamplerConfig * len(configs))(*configs)
    b = Batch(
        _ptr(logits), logits_stride if logits_stride is not None else logits.stride(0),
        _ptr(counts), (counts_stride if counts_stride is not None
                       else (counts.stride(0) if counts is not None else 0)),
        _ptr(uniforms), rows, _ptr(tokens), _ptr(token_logits), _ptr(row_status),
        _ptr(penalised), logprobs, _ptr(logprob_values), _ptr(logprob_ids))
    err = FgError()
    _check(lib().fg_sampler_hip_sample_static(vocab, arr, flags, C.byref(b), _stream(stream),
                                              C.byref(err)), err)


def plan(vocab: int, rows: int, traits: int = 0) -> Geometry:
    """Launch geometry of fg_sampler_hip_sample (host only, no device)."""
    g, err = Geometry(), FgError()
    _check(lib().fg_sampler_hip_plan(vocab, rows, traits, C.byref(g), C.byref(err)), err)
    return g


def block(g: Geometry, vocab: int, rows: int, b: int, wave: int):
    """(row, chunk, begin, end) of wave `wave` of workgroup `b` (host only)."""
    out = [C.c_uint32() for _ in range(4)]
    err = FgError()
    _check(lib().fg_sampler_hip_block(C.byref(g), vocab, rows, b, wave,
                                      *[C.byref(o) for o in out], C.byref(err)), err)
    return tuple(o.value for o in out)


def env_summary() -> dict:
    return {"lib": str(LIB_PATH), "exists": LIB_PATH.exists(),
            "target_groups": os.environ.get("FG_HIP_TARGET_GROUPS"),
            "paired": os.environ.get("FG_HIP_PAIRED"),
            "front_share": os.environ.get("FG_HIP_FRONT_SHARE"),
            "pace": os.environ.get("FG_HIP_PACE"),
            "finisher": os.environ.get("FG_HIP_FINISHER")}
