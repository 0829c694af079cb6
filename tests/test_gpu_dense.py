"""GPU parity of the Q8_0 cooked matrix-vector product (the LM head) and of
its fused greedy-finalist form.

Tolerance: the device sums in f32 in its own order, so each output is
checked against the exact f64 product with |y - y64| <= 1e-6 * sum|w x|
(the sum of magnitudes bounds any f32 summation's error; observed errors are
far below).  The reference's own test (tests/test_fg_vk.c:393-404) is also
restated with its own bound, 2e-4 * max(1, |ref|) against its f32 loop.  The
fused finalist must equal, bit for bit, the best (value, id) of the plain
kernel's output in fg_output_better's order."""
import numpy as np
import pytest

import fg_hip
import oracle_ffi as O

pytestmark = pytest.mark.gpu
TOL = 1e-6


def packed_random(rng, width, rows, scale_lo=1e-3, scale_hi=2e-2):
    """Random Q8_0 rows: uniform int8 quants, binary16 scales in a range."""
    blocks = width // 32
    b = rng.integers(0, 256, (rows, blocks, 34), dtype=np.uint8)
    d = rng.uniform(scale_lo, scale_hi, (rows, blocks)).astype(np.float16)
    b[:, :, :2] = d.view(np.uint8).reshape(rows, blocks, 2)
    return b.reshape(-1)


def to_dev(a, dev, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a))
    return t.to(dev) if dtype is None else t.to(dtype).to(dev)


def plain(dev, cooked, x, width, rows, scale):
    import torch
    tokens = x.shape[0]
    y = torch.empty(tokens * rows, dtype=torch.float32, device=dev)
    fg_hip.dense_q8_0_cooked(y, to_dev(cooked, dev), to_dev(x.astype(np.float32), dev), width,
                             rows, tokens, scale)
    torch.cuda.synchronize()
    return y.cpu().numpy().reshape(tokens, rows)


def check_f64(y, packed, x, width, rows, scale, sample=None):
    if sample is not None:
        blocks = width // 32
        sub = packed.reshape(rows, blocks * 34)[sample].reshape(-1)
        want, mag = O.dense_q8_0_f64(sub, x, width, len(sample), scale)
        y = y[:, sample]
    else:
        want, mag = O.dense_q8_0_f64(packed, x, width, rows, scale)
    err = np.abs(y.astype(np.float64) - want)
    assert np.all(err <= TOL * mag + 1e-30), float(np.max(err / (mag + 1e-30)))
    return float(np.max(err / (mag + 1e-30)))


def test_reference_cooked_dense_case(dev):
    """tests/test_fg_vk.c:393-404: 320 inputs, 17 rows, 2 tokens, scale 0.75,
    sin/cos data quantized by fg_quantize_q8_0."""
    width, rows, tokens = 320, 17, 2
    x = np.array([[np.cos(np.float32((t + 1) * (i + 5)) * np.float32(0.011)) for i in range(width)]
                  for t in range(tokens)], dtype=np.float32)
    src = np.array([np.sin(np.float32(i) * np.float32(0.007)) for i in range(width * rows)],
                   dtype=np.float32)
    packed = np.concatenate([fg_hip.quantize_q8_0(src[r * width:(r + 1) * width])
                             for r in range(rows)])
    cooked = fg_hip.cook_q8_0(packed, width, rows)
    got = plain(dev, cooked, x, width, rows, 0.75)
    ref = O.dense_q8_0_f32_reference_loop(packed, x, width, rows, 0.75)
    assert np.all(np.abs(got - ref) <= 2e-4 * np.maximum(1.0, np.abs(ref)))
    check_f64(got, packed, x, width, rows, 0.75)


@pytest.mark.parametrize("width,rows,tokens", [(32, 1, 1), (64, 17, 3), (2560, 1000, 1),
                                               (2560, 4099, 2), (4096, 300, 5), (8192, 50, 1),
                                               (96, 33, 4), (2560, 500, 7)])
def test_dense_matches_f64(dev, width, rows, tokens):
    rng = np.random.default_rng(width * 7 + rows)
    packed = packed_random(rng, width, rows)
    x = rng.normal(0, 1, (tokens, width)).astype(np.float32)
    cooked = fg_hip.cook_q8_0(packed, width, rows)
    got = plain(dev, cooked, x, width, rows, 1.25)
    worst = check_f64(got, packed, x, width, rows, 1.25)
    print(f"width {width} rows {rows} tokens {tokens}: worst |err|/sum|wx| {worst:.2e}")


def fused(dev, sl, cooked_slice, x, width, logits=True):
    import torch
    tokens = x.shape[0]
    v = torch.empty(tokens, dtype=torch.float32, device=dev)
    i = torch.empty(tokens, dtype=torch.int32, device=dev)
    s = torch.empty(tokens, dtype=torch.int32, device=dev)
    y = torch.empty(tokens * sl.rows, dtype=torch.float32, device=dev) if logits else None
    sl.run_dense(to_dev(cooked_slice, dev), to_dev(x.astype(np.float32), dev), width, tokens,
                 v, i, s, logits=y)
    torch.cuda.synchronize()
    return (v.cpu().numpy(), i.cpu().numpy().view(np.uint32), s.cpu().numpy(),
            None if y is None else y.cpu().numpy().reshape(tokens, sl.rows))


@pytest.mark.parametrize("ways,way,width,vocab,tokens", [(4, 1, 320, 4096, 3), (2, 1, 2560, 4000, 2),
                                                         (1, 0, 64, 1000, 1), (4, 3, 96, 999, 4),
                                                         (2, 0, 2560, 3000, 7)])
def test_fused_finalist_is_best_of_plain(dev, ways, way, width, vocab, tokens):
    rng = np.random.default_rng(ways * 100 + width)
    per = (vocab // ways) // 16 * 16
    first = per * way
    rows = per if way + 1 < ways else vocab - first
    packed = packed_random(rng, width, vocab)
    x = rng.normal(0, 1, (tokens, width)).astype(np.float32)
    blocks = width // 32
    slice_packed = packed.reshape(vocab, blocks * 34)[first:first + rows].reshape(-1)
    cooked = fg_hip.cook_q8_0(slice_packed, width, rows)
    ref = plain(dev, cooked, x, width, rows, 1.0)
    sl = fg_hip.OutputSlice(vocab, ways, first, rows, 8)
    for _ in range(2):  # the workspace returns to zero between calls
        v, i, s, y = fused(dev, sl, cooked, x, width)
        assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))
        wv, wi, ws = O.slice_finalists(ref, first)
        assert np.array_equal(i, wi) and np.array_equal(v.view(np.uint32), wv.view(np.uint32))
        assert np.array_equal(s, ws)
    v2, i2, _, _ = fused(dev, sl, cooked, x[:1], width, logits=False)
    assert i2[0] == i[0] and v2[0] == v[0]


@pytest.mark.parametrize("kind", ["zero_input", "nan_input", "inf_scale_row"])
def test_fused_finalist_special_values(dev, kind):
    """Zero and non-finite winners are recomputed from their tile: the fused
    value keeps the exact bits the plain kernel writes (sign of zero, NaN)."""
    rng = np.random.default_rng(5)
    width, rows = 128, 200
    packed = packed_random(rng, width, rows)
    x = rng.normal(0, 1, (2, width)).astype(np.float32)
    if kind == "zero_input":
        x[:] = 0.0
    elif kind == "nan_input":
        x[1, 7] = np.nan
    else:
        b = packed.reshape(rows, width // 32, 34)
        b[37, 2, :2] = np.array([0x00, 0x7c], dtype=np.uint8)  # scale +inf in row 37
    cooked = fg_hip.cook_q8_0(packed, width, rows)
    ref = plain(dev, cooked, x, width, rows, 1.0)
    sl = fg_hip.OutputSlice(rows, 1, 0, rows, 2)
    v, i, s, _ = fused(dev, sl, cooked, x, width)
    wv, wi, ws = O.slice_finalists(ref, 0)
    assert np.array_equal(i, wi) and np.array_equal(v.view(np.uint32), wv.view(np.uint32))
    assert np.array_equal(s, ws)
    if kind == "zero_input":
        assert np.all(i == 0) and np.all(s == 0)
    if kind == "nan_input":
        assert s[1] == 5 and np.isnan(v[1]) and s[0] == 0


def test_lm_head_full_shape(dev):
    """The reference's LM head shape (248,320 x 2,560, one token): fused
    finalist = best of the plain output; 4,096 sampled rows within the f64
    bound; the token is the f64 argmax unless the top two are within it."""
    import torch
    rng = np.random.default_rng(2560)
    width, vocab = 2560, 248320
    packed = packed_random(rng, width, vocab)
    cooked = fg_hip.cook_q8_0(packed, width, vocab)
    x = rng.normal(0, 1, (1, width)).astype(np.float32)
    ref = plain(dev, cooked, x, width, vocab, 1.0)
    sl = fg_hip.OutputSlice(vocab, 1, 0, vocab, 1)
    v, i, s, _ = fused(dev, sl, cooked, x, width, logits=False)
    wv, wi, _ = O.slice_finalists(ref, 0)
    assert i[0] == wi[0] and v[0] == wv[0] and s[0] == 0
    sample = np.sort(np.concatenate([rng.choice(vocab, 4096, replace=False),
                                     np.argsort(ref[0])[-8:]]))
    sample = np.unique(sample)
    check_f64(ref, packed, x, width, vocab, 1.0, sample=sample)
    top = np.argsort(ref[0])[-8:]
    want, mag = O.dense_q8_0_f64(packed.reshape(vocab, -1)[top].reshape(-1), x, width, 8, 1.0)
    order = np.argsort(-want[0])
    if want[0, order[0]] - want[0, order[1]] > 2 * TOL * mag[0].max():
        assert i[0] == top[order[0]]
    del cooked
    torch.cuda.empty_cache()


def test_dense_arguments(dev):
    import torch
    z = torch.zeros(4096, device=dev)
    for width in (0, 33, 16384 + 32):
        with pytest.raises(fg_hip.FgStatusError) as e:
            fg_hip.dense_q8_0_cooked(z, z, z, width, 4, 1)
        assert e.value.message.startswith("invalid cooked Q8_0 dense dispatch")
    sl = fg_hip.OutputSlice(4096, 4, 8, 1016, 2)  # not on a 16-row tile
    v = torch.empty(2, device=dev)
    with pytest.raises(fg_hip.FgStatusError):
        sl.run_dense(z, z, 32, 1, v, v, v)
