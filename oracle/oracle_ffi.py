"""ctypes binding of the CPU oracle (oracle/_build/libfg_oracle.so) and of the
reference's own sampler built from its sources (oracle/_ref/libfg_ref_sampler.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker and the timed CPU baseline.  The
product library never imports it.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_LIB = HERE / "_build" / "libfg_oracle.so"
REF_LIB = HERE / "_ref" / "libfg_ref_sampler.so"
REF_TEST = HERE / "_ref" / "test_sampler_ref"
INVALID_ID = 0xFFFFFFFF


class Config(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("top_k", C.c_uint32),
                ("presence", C.c_float), ("frequency", C.c_float), ("repetition", C.c_float)]


class Result(C.Structure):
    _fields_ = [("token", C.c_uint32), ("logit", C.c_float), ("status", C.c_int32),
                ("cutoff", C.c_uint32), ("margin", C.c_double)]


class RefConfig(C.Structure):
    """fg_sampler_config layout, for the reference library."""
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("top_k", C.c_uint32),
                ("presence_penalty", C.c_float), ("frequency_penalty", C.c_float),
                ("repetition_penalty", C.c_float), ("min_p", C.c_float), ("seed", C.c_uint64)]


class RefError(C.Structure):
    _fields_ = [("code", C.c_int), ("message", C.c_char * 512)]


_O = None
_R = None


def _p(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


def oracle() -> C.CDLL:
    global _O
    if _O is None:
        if not ORACLE_LIB.exists():
            raise RuntimeError(f"oracle not built: {ORACLE_LIB}")
        o = C.CDLL(str(ORACLE_LIB))
        P, u32, u64, f32, f64 = C.c_void_p, C.c_uint32, C.c_uint64, C.c_float, C.c_double
        sig = {
            "fgo_philox4x32_10": (None, [P, P, P]),
            "fgo_xorshift_uniform": (f32, [C.POINTER(u64)]),
            "fgo_float_key": (u32, [f32]),
            "fgo_penalties_c": (None, [P, P, u32, f32, f32, f32]),
            "fgo_penalties_glsl": (None, [P, P, u32, f32, f32, f32]),
            "fgo_greedy_before": (C.c_int, [f32, u32, f32, u32]),
            "fgo_argmax_reduce_step": (u32, [P, P, P, P, u32]),
            "fgo_topk_select_step": (u32, [P, P, P, P, u32, u32]),
            "fgo_topk_row": (u32, [P, u32, u32, P, P]),
            "fgo_select": (C.c_int32, [f32, f32, u32, P, P, u32, f32, P, P, P, P]),
            "fgo_sample_rows": (C.c_int, [P, P, u64, P, u64, u32, P, u32, u32, P, P, P, P, u32]),
            "fgo_u01": (f64, [u32]),
            "fgo_gen_uniforms": (None, [P, u32, u32, u32]),
            "fgo_gen_logits": (None, [P, u64, u32, u32, C.c_int, f64, f64, f64, u32, u32]),
            "fgo_gen_zipf_ids": (None, [P, u32, u32, u32, f64, u32, u32]),
            "fgo_gen_uniform_ids": (None, [P, u32, u32, u32, u32, u32]),
            "fgo_build_counts": (None, [P, u64, u32, u32, P, u32]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(o, name)
            fn.restype = res
            fn.argtypes = args
        _O = o
    return _O


def reference_available() -> bool:
    return REF_LIB.exists()


def reference() -> C.CDLL:
    global _R
    if _R is None:
        r = C.CDLL(str(REF_LIB))
        P, u32, f32 = C.c_void_p, C.c_uint32, C.c_float
        r.fg_sampler_select.restype = C.c_int
        r.fg_sampler_select.argtypes = [C.POINTER(RefConfig), P, P, u32, f32, P, P,
                                        C.POINTER(RefError)]
        r.fg_sampler_apply_penalties.restype = None
        r.fg_sampler_apply_penalties.argtypes = [P, P, P, u32, C.POINTER(RefConfig)]
        r.fg_sampler_uniform.restype = f32
        r.fg_sampler_uniform.argtypes = [P]
        r.fg_sampler_state_init.restype = None
        r.fg_sampler_state_init.argtypes = [P, C.c_uint64]
        r.fg_sampler_config_validate.restype = C.c_int
        r.fg_sampler_config_validate.argtypes = [C.POINTER(RefConfig), C.POINTER(RefError)]
        _R = r
    return _R


# ---- numpy helpers -----------------------------------------------------------

def philox(ctr, key):
    c = np.asarray(ctr, dtype=np.uint32)
    k = np.asarray(key, dtype=np.uint32)
    out = np.zeros(4, dtype=np.uint32)
    oracle().fgo_philox4x32_10(_p(c), _p(k), _p(out))
    return out


def gen_logits(rows, n, kind, sigma, sigma2=0.0, nu=0.0, seed=1, config_id=0):
    out = np.zeros((rows, n), dtype=np.float32)
    oracle().fgo_gen_logits(_p(out), n, rows, n, kind, sigma, sigma2, nu, seed, config_id)
    return out


def gen_uniforms(rows, seed, config_id):
    out = np.zeros(rows, dtype=np.float32)
    oracle().fgo_gen_uniforms(_p(out), rows, seed, config_id)
    return out


def gen_zipf_ids(rows, per_row, n, s, seed, config_id):
    out = np.zeros((rows, per_row), dtype=np.uint32)
    oracle().fgo_gen_zipf_ids(_p(out), rows, per_row, n, s, seed, config_id)
    return out


def gen_uniform_ids(rows, per_row, n, seed, config_id):
    out = np.zeros((rows, per_row), dtype=np.uint32)
    oracle().fgo_gen_uniform_ids(_p(out), rows, per_row, n, seed, config_id)
    return out


def build_counts(ids, n):
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    rows, per_row = ids.shape
    out = np.zeros((rows, n), dtype=np.uint32)
    oracle().fgo_build_counts(_p(out), n, rows, n, _p(ids), per_row)
    return out


def penalties_c(scores, counts, presence, frequency, repetition):
    s = np.ascontiguousarray(scores, dtype=np.float32).copy()
    c = np.ascontiguousarray(counts, dtype=np.uint32)
    oracle().fgo_penalties_c(_p(s), _p(c), s.size, presence, frequency, repetition)
    return s


def penalties_glsl(scores, counts, presence, frequency, repetition):
    s = np.ascontiguousarray(scores, dtype=np.float32).copy()
    c = np.ascontiguousarray(counts, dtype=np.uint32)
    oracle().fgo_penalties_glsl(_p(s), _p(c), s.size, presence, frequency, repetition)
    return s


def argmax_reduce_step(scores, ids=None):
    s = np.ascontiguousarray(scores, dtype=np.float32)
    i = None if ids is None else np.ascontiguousarray(ids, dtype=np.uint32)
    groups = (s.size + 4095) // 4096
    os_ = np.zeros(groups, dtype=np.float32)
    oi = np.zeros(groups, dtype=np.uint32)
    oracle().fgo_argmax_reduce_step(_p(os_), _p(oi), _p(s), _p(i), s.size)
    return os_, oi


def topk_select_step(scores, k, ids=None):
    s = np.ascontiguousarray(scores, dtype=np.float32)
    i = None if ids is None else np.ascontiguousarray(ids, dtype=np.uint32)
    tiles = (s.size + 1023) // 1024
    os_ = np.zeros(tiles * k, dtype=np.float32)
    oi = np.zeros(tiles * k, dtype=np.uint32)
    oracle().fgo_topk_select_step(_p(os_), _p(oi), _p(s), _p(i), s.size, k)
    return os_, oi


def topk_row(scores, k):
    s = np.ascontiguousarray(scores, dtype=np.float32)
    os_ = np.zeros(k, dtype=np.float32)
    oi = np.zeros(k, dtype=np.uint32)
    have = oracle().fgo_topk_row(_p(s), s.size, k, _p(os_), _p(oi))
    return os_, oi, have


def select(temperature, top_p, top_k, scores, ids, uniform):
    s = np.ascontiguousarray(scores, dtype=np.float32)
    i = np.ascontiguousarray(ids, dtype=np.uint32)
    tok, logit, cut, margin = C.c_uint32(), C.c_float(), C.c_uint32(), C.c_double()
    st = oracle().fgo_select(temperature, top_p, top_k, _p(s), _p(i), s.size, uniform,
                             C.byref(tok), C.byref(logit), C.byref(cut), C.byref(margin))
    return st, tok.value, logit.value, cut.value, margin.value


def sample_rows(configs, logits, uniforms, counts=None, logprobs=0, want_penalised=False,
                threads=1):
    """configs: list of dicts with temperature/top_p/top_k/presence/frequency/repetition."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    rows, n = logits.shape
    cfg = (Config * rows)(*[Config(c["temperature"], c["top_p"], c["top_k"], c.get("presence", 0.0),
                                   c.get("frequency", 0.0), c.get("repetition", 1.0))
                            for c in configs])
    res = (Result * rows)()
    u = np.ascontiguousarray(uniforms, dtype=np.float32)
    cnt = None if counts is None else np.ascontiguousarray(counts, dtype=np.uint32)
    lpv = np.zeros((rows, max(logprobs, 1)), dtype=np.float32)
    lpi = np.zeros((rows, max(logprobs, 1)), dtype=np.uint32)
    pen = np.zeros((rows, n), dtype=np.float32) if want_penalised else None
    oracle().fgo_sample_rows(cfg, _p(logits), n, _p(cnt), n if cnt is not None else 0, n,
                             _p(u), rows, logprobs, res, _p(lpv), _p(lpi), _p(pen), threads)
    out = {
        "token": np.array([r.token for r in res], dtype=np.uint32),
        "logit": np.array([r.logit for r in res], dtype=np.float32),
        "status": np.array([r.status for r in res], dtype=np.int32),
        "cutoff": np.array([r.cutoff for r in res], dtype=np.uint32),
        "margin": np.array([r.margin for r in res], dtype=np.float64),
    }
    if logprobs:
        out["lp_values"] = lpv[:, :logprobs]
        out["lp_ids"] = lpi[:, :logprobs]
    if want_penalised:
        out["penalised"] = pen
    return out


# ---- output-history payload (restatement; pinned by tests/golden/ref_history_vectors.json) ----

HISTORY_HEADER = 8
HISTORY_MAX_COUNT = 262144  # FG_NATIVE_CONTEXT
HISTORY_MAX_SLOTS = 2       # FG_DECODE_BATCH_MAX_SLOTS


def history_decode(payload: bytes, capacity: int, vocab: int):
    """fg_output_history_decode (reference src/protocol.c:1348-1366) restated:
    returns (status, tokens, slot); status 2 = FG_ERR_ARGUMENT (shorter than
    the header), 4 = FG_ERR_FORMAT (reserved bytes, slot, count vs context,
    capacity and size, token range), 0 = OK."""
    if len(payload) < HISTORY_HEADER:
        return 2, None, None
    count = int.from_bytes(payload[0:4], "big")
    slot = payload[4]
    reserved = int.from_bytes(payload[5:8], "big")
    if (reserved or slot >= HISTORY_MAX_SLOTS or count > HISTORY_MAX_COUNT or count > capacity
            or HISTORY_HEADER + 4 * count != len(payload)):
        return 4, None, None
    tokens = [int.from_bytes(payload[HISTORY_HEADER + 4 * i:HISTORY_HEADER + 4 * i + 4], "big")
              for i in range(count)]
    if any(t >= vocab for t in tokens):
        return 4, None, None
    return 0, tokens, slot


# ---- top-512 tile reduction (restatement of shaders/fg_topk_reduce_v2.comp) ----

REDUCE_TILE = 4096
REDUCE_KEEP = 512


def reduce_before(a: float, ai: int, b: float, bi: int) -> bool:
    """The comparator of shaders/fg_topk_reduce_v2.comp:9 (also
    tests/test_fg_vk.c:1223-1229): padding id 0xffffffff last; non-finite
    first, lower id first among them; then larger value, lower id on ties."""
    ap, bp = ai == 0xFFFFFFFF, bi == 0xFFFFFFFF
    if ap or bp:
        return (not ap) and bp
    an, bn = not np.isfinite(a), not np.isfinite(b)
    if an or bn:
        return an if an != bn else ai < bi
    return a > b or (a == b and ai < bi)


def reduce_order_key(scores: np.ndarray, ids: np.ndarray):
    """np.lexsort keys (last = primary) giving the comparator's order."""
    s = scores.astype(np.float64)
    pad = (ids == 0xFFFFFFFF).astype(np.int64)
    nonfinite = ~np.isfinite(s)
    value = np.where(nonfinite, 0.0, s)
    return (ids.astype(np.int64), -value, (~nonfinite).astype(np.int64), pad)


def topk_reduce_step(scores: np.ndarray, ids: np.ndarray):
    """fg_vk_topk_reduce (src/vk.c:2235) restated: per 4096-value tile the
    entries in comparator order, the first min(512, n) kept, the rest of the
    512 slots (-inf, 0xffffffff); a single tile with fewer than 512 values
    yields exactly `count` entries."""
    count = scores.size
    tiles = (count + REDUCE_TILE - 1) // REDUCE_TILE
    produced = count if tiles == 1 and count < REDUCE_KEEP else tiles * REDUCE_KEEP
    per = produced if tiles == 1 else REDUCE_KEEP
    out_s = np.full(produced, -np.inf, dtype=np.float32)
    out_i = np.full(produced, 0xFFFFFFFF, dtype=np.uint32)
    for g in range(tiles):
        s = scores[g * REDUCE_TILE:(g + 1) * REDUCE_TILE]
        i = ids[g * REDUCE_TILE:(g + 1) * REDUCE_TILE]
        order = np.lexsort(reduce_order_key(s, i))
        keep = order[:min(REDUCE_KEEP, s.size, per)]
        out_s[g * per:g * per + keep.size] = s[keep]
        out_i[g * per:g * per + keep.size] = i[keep]
    return out_s, out_i


# ---- vocabulary-split greedy output ------------------------------------------

SPLIT_RANKS = (4, 0, 1, 2)  # way -> rank, src/protocol.c:23-44
STATUS_MISMATCH = 5


def output_better(a: float, ai: int, b: float, bi: int) -> bool:
    """fg_output_better (src/output.c:484-492): the same order as the top-512
    reduction's comparator."""
    return reduce_before(a, ai, b, bi)


def slice_finalists(logits: np.ndarray, first_row: int):
    """The reduction of fg_output_slice_run (src/output.c:320-344) per row of
    logits[rows, slice]: the best (value, id) in fg_output_better's order,
    ids first_row + i, status 5 (FG_ERR_MISMATCH) when the value is
    non-finite."""
    rows, n = logits.shape
    ids = np.arange(first_row, first_row + n, dtype=np.uint32)
    vals = np.empty(rows, dtype=np.float32)
    out = np.empty(rows, dtype=np.uint32)
    status = np.zeros(rows, dtype=np.int32)
    for r in range(rows):
        best = int(np.lexsort(reduce_order_key(logits[r], ids))[0])
        vals[r], out[r] = logits[r, best], ids[best]
        status[r] = 0 if np.isfinite(vals[r]) else STATUS_MISMATCH
    return vals, out, status


def split_combine_row(values, ids, ranks, ways: int, vocab: int, spans):
    """The owner's combine (src/runtime.c:2440-2466) for one row: entry 0 is
    the owner's finalist, entries 1.. come with their ranks; spans[w] =
    (first, rows).  Returns (status, token, value); token 0xffffffff on
    failure."""
    value, tid = float(np.float32(values[0])), int(ids[0])
    for i in range(1, ways):
        rank, rid = int(ranks[i]), int(ids[i])
        if rank not in SPLIT_RANKS[:ways]:
            return STATUS_MISMATCH, 0xFFFFFFFF, None
        first, n = spans[SPLIT_RANKS[:ways].index(rank)]
        if not first <= rid < first + n:
            return STATUS_MISMATCH, 0xFFFFFFFF, None
        if output_better(np.float32(values[i]), rid, value, tid):
            value, tid = float(np.float32(values[i])), rid
    if tid >= vocab or not np.isfinite(value):
        return STATUS_MISMATCH, 0xFFFFFFFF, value
    return 0, tid, value


# ---- Q8_0 cooked matrix-vector product ---------------------------------------

def q8_0_dequantize_rows(packed: np.ndarray, width: int, rows: int) -> np.ndarray:
    """Packed Q8_0 rows -> f64 [rows, width]: d (binary16, widened exactly) * q
    (src/quant.c:45-47; the product is exact in f64)."""
    blocks = width // 32
    b = np.asarray(packed, dtype=np.uint8).reshape(rows, blocks, 34)
    d = b[:, :, :2].copy().view(np.float16)[..., 0].astype(np.float64)
    q = b[:, :, 2:].view(np.int8).astype(np.float64)
    return (d[:, :, None] * q).reshape(rows, width)


def dense_q8_0_f64(packed: np.ndarray, x: np.ndarray, width: int, rows: int, scale: float):
    """scale * W x in f64 (exact products, f64 sums) for x [tokens, width];
    returns (y [tokens, rows], magnitude [tokens, rows] = scale * sum |w x|),
    the second bounding the f32 rounding error of any summation order."""
    w = q8_0_dequantize_rows(packed, width, rows)
    xs = np.asarray(x, dtype=np.float64)
    return (xs @ w.T) * scale, (np.abs(xs) @ np.abs(w).T) * abs(scale)


def dense_q8_0_f32_reference_loop(packed: np.ndarray, x: np.ndarray, width: int, rows: int,
                                  scale: float) -> np.ndarray:
    """The reference test's CPU product (tests/test_fg_vk.c:393-404): one f32
    fmaf chain per row over delta*q and x, times scale; small sizes only."""
    blocks = width // 32
    b = np.asarray(packed, dtype=np.uint8).reshape(rows, blocks, 34)
    d = b[:, :, :2].copy().view(np.float16)[..., 0].astype(np.float32)
    q = b[:, :, 2:].view(np.int8).astype(np.float32)
    x = np.asarray(x, dtype=np.float32)
    out = np.empty((x.shape[0], rows), dtype=np.float32)
    for t in range(x.shape[0]):
        for r in range(rows):
            acc = np.float32(0.0)
            for blk in range(blocks):
                for i in range(32):
                    wv = np.float32(d[r, blk] * q[r, blk, i])
                    acc = np.float32(float(wv) * float(x[t, blk * 32 + i]) + float(acc))
            out[t, r] = np.float32(acc * np.float32(scale))
    return out
