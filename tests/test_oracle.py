"""CPU tests that pin the oracle (oracle/qwref.c) to the reference.

Each check is either a known answer held by the reference's own tests (cited
file:line under /root/reference), a comparison with an independent
implementation (numpy float16, f64 brute force), or a closed form -- chosen so
that a plausible restatement mistake (a dropped term, a wrong sign or index, a
transposed operand) fails one of them.
"""
import math

import numpy as np
import pytest

from oracle import oracle as o
from util import lcg_values, normal


# ---------------------------------------------------------------- packing KAT
def test_quant_hash_matches_reference_golden():
    # selftest.zig:294 / tools/wasm_selftest.mjs:22: FNV-1a over the q4, q5, q8
    # planes of 128 values cos(i * 0.19) * 1.75.
    assert o.quant_hash() == 0xF247917B05691FD1


# ---------------------------------------------------------------- f16 codec
def test_f16_known_answers():
    # half_float.zig:47-68
    for v in [0.0, -0.0, 1.0, -1.0, 0.5, 2.0, 1024.0, 0.0009765625, 65504.0]:
        assert o.from_f16(o.to_f16(v)) == v
    assert o.from_f16(o.to_f16(1.0 + 1.0 / 2048.0)) == 1.0
    assert o.from_f16(o.to_f16(1.0 + 3.0 / 2048.0)) == 1.0 + 2.0 / 1024.0
    assert math.isinf(o.from_f16(o.to_f16(1.0e30))) and o.from_f16(o.to_f16(1.0e30)) > 0
    assert math.isinf(o.from_f16(o.to_f16(-1.0e30))) and o.from_f16(o.to_f16(-1.0e30)) < 0
    value = 1e-4
    while value < 1.0:
        assert abs(o.from_f16(o.to_f16(value)) - value) / value < 0.0005
        value *= 1.7


def test_f16_matches_numpy_round_to_nearest_even():
    # Independent implementation: numpy's float32 -> float16 cast (RNE,
    # subnormals, overflow to inf). Strided sweep over every f32 exponent.
    lib = o.lib()
    bits = np.arange(0, 1 << 32, 4099, dtype=np.uint64).astype(np.uint32)
    extra = np.array([0x33000000, 0x33000001, 0x387FC000, 0x387FE000, 0x38800000, 0x477FE000,
                      0x477FEFFF, 0x477FF000, 0x7F800000, 0xFF800000, 0x00000001, 0x80000000], np.uint32)
    bits = np.concatenate([bits, extra])
    values = bits.view(np.float32)
    finite = np.isfinite(values) | np.isinf(values)
    values = values[finite]
    with np.errstate(over="ignore"):
        expected = values.astype(np.float16).view(np.uint16)
    actual = np.array([lib.qwref_to_f16(float(v)) for v in values], np.uint16)
    mismatch = np.nonzero(actual != expected)[0]
    assert mismatch.size == 0, [(hex(values.view(np.uint32)[i]), hex(actual[i]), hex(expected[i])) for i in mismatch[:5]]


def test_f16_widening_is_exact_for_every_pattern():
    lib = o.lib()
    patterns = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    expected = patterns.view(np.float16).astype(np.float32)
    actual = np.array([lib.qwref_from_f16(int(p)) for p in patterns], np.float32)
    nan = np.isnan(expected)
    assert np.array_equal(np.isnan(actual), nan)
    assert np.array_equal(actual[~nan].view(np.uint32), expected[~nan].view(np.uint32))


def test_bf16_known_answers():
    # half_float.zig:79-111
    lib = o.lib()
    for v in [0.0, 1.0, -1.0, 0.5, 1.5, -0.25, 256.0, 1024.0, 65536.0]:
        assert lib.qwref_from_bf16(lib.qwref_to_bf16(v)) == v
    even = np.array([0x3F808000], np.uint32).view(np.float32)[0]
    assert lib.qwref_from_bf16(lib.qwref_to_bf16(float(even))) == 1.0
    odd = np.array([0x3F818000], np.uint32).view(np.float32)[0]
    assert lib.qwref_to_bf16(float(odd)) == 0x3F82


# ---------------------------------------------------------------- layout
def test_plane_layout_offsets():
    # quant.zig:423-448
    st, l = o.plane_layout(o.Q4, 896, 896, 0, 16)
    assert st == 0 and l.groups_per_row == 14 and l.group_count == 14 * 896
    assert l.scales_offset_bytes == 0 and l.scales_len_bytes == 14 * 896 * 2
    assert l.data_offset_bytes % 16 == 0 and l.data_len_bytes == 14 * 896 * 32
    assert l.total_len_bytes == l.data_offset_bytes + l.data_len_bytes
    st, l = o.plane_layout(o.Q5, 64, 256, 33, 16)
    assert (l.scales_offset_bytes, l.scales_len_bytes, l.group_count) == (15, 512, 256)
    assert (l.data_offset_bytes, l.data_len_bytes, l.total_len_bytes) == (527, 256 * 40, 10767)
    assert (33 + l.data_offset_bytes) % 16 == 0


def test_plane_layout_rejects_bad_arguments():
    # quant.zig:450-455 and :395-400
    assert o.plane_layout(o.Q4, 64, 64, 0, 2)[0] == -1
    assert o.plane_layout(200, 64, 64, 0, 16)[0] == -3
    assert o.plane_layout(o.Q4, 1, 100, 0, 16)[0] == -7


def test_kv_cache_bytes():
    # quant.zig:402-421
    f32 = 2 * 28 * o.plane_bytes(0, 8192, 1024)
    q8 = 2 * 28 * o.plane_bytes(o.Q8, 8192, 1024)
    assert f32 == 1879048192
    assert q8 // (2 * 28) == 8192 * (1024 + 16 * 2)
    assert q8 < f32 // 3


# ---------------------------------------------------------------- quantizer
def test_exact_values_survive_quantization():
    # quant.zig:527-542
    v = np.zeros(64, np.float32)
    v[0], v[1] = 7.0, -8.0
    s, d = o.quantize_rows(o.Q4, v)
    assert s.view(np.uint16)[0] == 0x3C00
    dec = o.dequantize_rows(o.Q4, s, d, 1, 64)[0]
    assert dec[0] == 7.0 and dec[1] == -8.0 and np.all(dec[2:] == 0.0)
    assert d[0] == 0x0F and d[1] == 0x88


def test_zero_group_stores_zero_scale_and_bias_codes():
    # quant.zig:544-554
    v = np.zeros(64, np.float32)
    for fmt, code in [(o.Q4, 0x88), (o.Q8, 0x80)]:
        s, d = o.quantize_rows(fmt, v)
        assert s.view(np.uint16)[0] == 0
        assert np.all(d[: o.DATA_BYTES[fmt]] == code)
        assert o.dot_row(fmt, s, d, v) == 0.0


@pytest.mark.parametrize("fmt", [o.Q4, o.Q5, o.Q8])
def test_round_trip_within_one_step(fmt):
    # quant.zig:457-498
    idx = np.arange(64, dtype=np.float32)
    v = (np.sin(idx * np.float32(0.37)) * np.float32(3.0) + idx * np.float32(0.01)).astype(np.float32)
    s, d = o.quantize_rows(fmt, v)
    dec = o.dequantize_rows(fmt, s, d, 1, 64)[0]
    bias = o.lib().qwref_bias(fmt)
    step = np.float32(np.abs(v).max()) / np.float32(bias)
    bound = step * (1.0 + bias * 0.00048828125) + 1e-6
    diff = np.abs(v.astype(np.float64) - dec)
    assert np.all(diff <= bound)
    assert math.sqrt(float(np.mean(diff ** 2))) <= step * 0.5


def test_error_shrinks_with_code_width():
    # quant.zig:500-525
    idx = np.arange(64, dtype=np.float32)
    v = (np.cos(idx * np.float32(0.53)) * np.float32(2.5) + np.sin(idx * np.float32(0.11))).astype(np.float32)
    previous = float("inf")
    for fmt in (o.Q4, o.Q5, o.Q8):
        s, d = o.quantize_rows(fmt, v)
        err = float(np.abs(v - o.dequantize_rows(fmt, s, d, 1, 64)[0]).sum())
        assert err < previous
        previous = err


def test_q5_bit_planes():
    # quant.zig:597-624
    v = np.zeros(64, np.float32)
    v[0], v[1] = 15.0, -16.0
    s, d = o.quantize_rows(o.Q5, v)
    dec = o.dequantize_rows(o.Q5, s, d, 1, 64)[0]
    assert dec[0] == 15.0 and dec[1] == -16.0 and np.all(dec[2:] == 0)
    assert d[0] == 0x0F
    assert d[32] & 0x01 and not d[32] & 0x02
    assert np.all(d[33:40] == 0xFF)


def test_quantizer_codes_follow_the_definition():
    # Independent restatement in f64-free numpy f32 arithmetic: scale =
    # f16(max/bias), code = round-half-away(v / stored) clamped.
    values = normal(64 * 40, 11).reshape(40, 64) * np.float32(0.3)
    values[3] = 0.0
    values[5, 7] = np.float32(1e-7)  # a subnormal-scale group
    values[5, :7] = 0.0
    values[5, 8:] = 0.0
    for fmt, bias in [(o.Q4, 8), (o.Q8, 128)]:
        s, d = o.quantize_rows(fmt, values)
        scale = (np.abs(values).max(axis=1) / np.float32(bias)).astype(np.float16)
        assert np.array_equal(s.view(np.uint16), scale.view(np.uint16))
        stored = scale.astype(np.float32)[:, None]
        with np.errstate(divide="ignore", invalid="ignore"):
            scaled = np.where(stored == 0, np.float32(0), values / stored).astype(np.float32)
        rounded = np.where(scaled >= 0, np.floor(scaled + np.float32(0.5)), np.ceil(scaled - np.float32(0.5)))
        codes = (np.clip(rounded, -bias, bias - 1) + bias).astype(np.uint8)
        if fmt == o.Q4:
            packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
            assert np.array_equal(d, packed.reshape(-1))
        else:
            assert np.array_equal(d, codes.reshape(-1))


# ---------------------------------------------------------------- linear
def test_matrix_dispatch_ones_row_is_56():
    # kernels.zig:932-971: scale 1/8, code 7 -> 0.875 each, 64 of them.
    ones = np.ones(64, np.float32)
    s, d = o.quantize_rows(o.Q4, ones)
    assert o.linear_quantized(o.Q4, s, d, 1, 64, ones)[0, 0] == 56.0


def test_dot_row_agrees_with_dense():
    # quant.zig:575-595
    idx = np.arange(256, dtype=np.float32)
    v = (np.cos(idx * np.float32(0.11)) * np.float32(1.5)).astype(np.float32)
    x = (np.sin(idx * np.float32(0.07)) * np.float32(0.5)).astype(np.float32)
    s, d = o.quantize_rows(o.Q4, v)
    dense = o.dequantize_rows(o.Q4, s, d, 1, 256)[0]
    expected = np.float32(0)
    for w, a in zip(dense, x):
        expected = np.float32(expected + np.float32(w * a))
    assert abs(o.dot_row(o.Q4, s, d, x) - expected) <= 1e-5 * abs(expected)


def test_linear_f32_hand_computed():
    # kernels.zig:840-850
    out = o.linear_f32(np.array([[1, 0, 0], [0, 1, 1]], np.float32), np.array([1, 2, 3, 4, 5, 6], np.float32), 2)
    assert out.tolist() == [[1.0, 5.0], [4.0, 11.0]]


def test_matrix_dispatch_every_storage_kind():
    # kernels.zig:932-948: 2 x 64 ones against ones give 64 for f32 and f16.
    x = np.ones(64, np.float32)
    assert o.linear_f32(np.ones((2, 64), np.float32), x).tolist() == [[64.0, 64.0]]
    ones_f16 = np.full((2, 64), o.to_f16(1.0), np.uint16)
    assert o.linear_f16(ones_f16, x).tolist() == [[64.0, 64.0]]


def test_f16_and_f32_linear_agree_on_exact_weights():
    # kernels.zig:863-876: two tokens of four columns; weights exact in f16,
    # so linearF16 equals linearF32, and every sum here is exact in f32.
    x = np.array([0.5, -1.5, 2.0, 1.0, -0.5, 0.25, 1.0, -2.0], np.float32)
    w = np.array([[2.0, 0.5, -1.0, 0.0], [1.0, 1.0, 0.5, -2.0]], np.float32)
    bits = np.array([[o.to_f16(float(v)) for v in row] for row in w], np.uint16)
    out32 = o.linear_f32(w, x, 2)
    assert np.array_equal(o.linear_f16(bits, x, 2), out32)
    assert out32.tolist() == [[-1.75, -2.0], [-1.875, 4.25]]


@pytest.mark.parametrize("rows,cols,tokens", [(5, 67, 3), (9, 256, 2), (3, 1, 4)])
def test_linear_f16_against_numpy_widening_and_f64(rows, cols, tokens):
    # Every finite f16 class (subnormals, the largest normal, both signs):
    # numpy's own f16 -> f32 widening then the f32 linear must agree bit for
    # bit, and the result must sit within f32 rounding of the f64 product.
    rng = np.random.default_rng(rows * 1000 + cols)
    bits = rng.integers(0, 1 << 16, size=(rows, cols), dtype=np.uint16)
    bits[(bits & 0x7C00) == 0x7C00] &= 0x83FF  # inf / NaN -> subnormals
    bits.flat[0] = 0x7BFF  # 65504
    bits.flat[-1] = 0x0001  # the smallest subnormal
    x = (normal(tokens * cols, 5, 3) * np.float32(1e-3)).reshape(tokens, cols)
    widened = bits.view(np.float16).astype(np.float32)
    actual = o.linear_f16(bits, x, tokens)
    assert np.array_equal(actual, o.linear_f32(widened, x, tokens))
    expected = x.astype(np.float64) @ widened.astype(np.float64).T
    scale = np.abs(x.astype(np.float64)) @ np.abs(widened.astype(np.float64)).T
    assert np.all(np.abs(actual - expected) <= 1e-6 * scale + 1e-30)


def test_embedding_row_every_storage_kind():
    # decoder.zig:378-420: sin(0.03 i) over 3 x 64 values; f32 rows exact,
    # f16 rows within 1e-3 (and numpy's widening of the same bits exactly),
    # q4 rows within 0.2; decoder.zig:423-435: a row past the end is refused.
    cols, rows = 64, 3
    values = np.sin(np.arange(rows * cols, dtype=np.float32) * np.float32(0.03)).astype(np.float32)
    m = values.reshape(rows, cols)
    assert np.array_equal(o.embedding_row(o.F32, None, values, rows, cols, 1), m[1])
    bits = np.array([o.to_f16(float(v)) for v in values], np.uint16)
    got = o.embedding_row(o.F16, None, bits, rows, cols, 2)
    assert np.max(np.abs(got - m[2])) <= 1e-3
    assert np.array_equal(got, bits.reshape(rows, cols)[2].view(np.float16).astype(np.float32))
    s, d = o.quantize_rows(o.Q4, m)
    assert np.max(np.abs(o.embedding_row(o.Q4, s, d, rows, cols, 1) - m[1])) <= 0.2
    with pytest.raises(ValueError):
        o.embedding_row(o.F32, None, np.zeros(64, np.float32), 1, cols, 1)


def test_linear_shape_mismatch():
    s, d = o.quantize_rows(o.Q4, np.ones((2, 64), np.float32))
    lib = o.lib()
    out = np.zeros(2, np.float32)
    x = np.ones(64, np.float32)
    assert lib.qwref_linear_quantized(out.ctypes.data, x.ctypes.data, o.Q4, s.ctypes.data, s.size - 2,
                                      d.ctypes.data, d.size, 2, 64, 1) == -7
    assert lib.qwref_linear_quantized(out.ctypes.data, x.ctypes.data, o.Q4, s.ctypes.data, s.size,
                                      d.ctypes.data, d.size, 2, 100, 1) == -7


@pytest.mark.parametrize("fmt,rows,cols,tokens", [(o.Q4, 37, 192, 3), (o.Q8, 19, 320, 2), (o.Q5, 8, 128, 1)])
def test_linear_quantized_against_f64_brute_force(fmt, rows, cols, tokens):
    w = normal(rows * cols, 21, 1, 0.02).reshape(rows, cols)
    x = normal(tokens * cols, 21, 2).reshape(tokens, cols)
    s, d = o.quantize_rows(fmt, w)
    dense = o.dequantize_rows(fmt, s, d, rows, cols).astype(np.float64)
    # dequant is exact: f32(u - bias) * f16 scale (8-bit x 11-bit significands)
    gpr = cols // 64
    sc = s.view(np.float16).astype(np.float64).reshape(rows, gpr)
    approx = dense / np.repeat(np.where(sc == 0, 1, sc), 64, axis=1)
    assert np.array_equal(approx, np.round(approx))
    expected = x.astype(np.float64) @ dense.T
    actual = o.linear_quantized(fmt, s, d, rows, cols, x, tokens)
    scale = np.abs(x.astype(np.float64)) @ np.abs(dense.T)
    assert np.all(np.abs(actual - expected) <= 1e-6 * scale + 1e-12)


def test_dot_f32_lane_order():
    # kernels.zig:39-51: four lanes (j, j+4, ...), reduced in lane order, then
    # a scalar tail. Values chosen so that another order rounds differently.
    a = np.array([1e8, 1.0, -1e8, 1.0, 1.0, 1.0, 1.0, 1.0, 3.0], np.float32)
    b = np.ones(9, np.float32)
    lanes = [np.float32(0)] * 4
    for i in range(8):
        lanes[i % 4] = np.float32(lanes[i % 4] + a[i] * b[i])
    total = np.float32(np.float32(np.float32(lanes[0] + lanes[1]) + lanes[2]) + lanes[3])
    total = np.float32(total + a[8] * b[8])
    assert o.dot_f32(a, b) == total


# ---------------------------------------------------------------- attention
def _q8_planes(rows: np.ndarray):
    s, d = o.quantize_rows(o.Q8, rows)
    return s, d


def test_q8_attention_agrees_with_f32_attention():
    # kernels.zig:769-836, the reference's own LCG inputs and 0.05 bound.
    head_dim, kvh, heads, cached = 64, 2, 4, 5
    kvw = kvh * head_dim
    keys, state = lcg_values(cached * kvw, 7, 200.0)
    values, state = lcg_values(cached * kvw, state, 400.0)
    query, state = lcg_values(heads * head_dim, state, 500.0)
    ks, kc = _q8_planes(keys.reshape(cached, kvw))
    vs, vc = _q8_planes(values.reshape(cached, kvw))
    exact = o.decode_attention(query, keys, values, cached, heads, kvh, head_dim)
    quant = o.decode_attention_q8(query, ks, kc, vs, vc, cached, heads, kvh, head_dim)
    assert np.all(np.abs(exact - quant) <= 0.05)


def _attention_f64(query, k_deq, v_deq, heads, kvh, head_dim):
    groups = heads // kvh
    out = np.zeros(heads * head_dim)
    for h in range(heads):
        g = h // groups
        q = query[h * head_dim:(h + 1) * head_dim].astype(np.float64)
        kk = k_deq[:, g * head_dim:(g + 1) * head_dim]
        vv = v_deq[:, g * head_dim:(g + 1) * head_dim]
        sc = kk @ q / math.sqrt(head_dim)
        p = np.exp(sc - sc.max())
        p /= p.sum()
        out[h * head_dim:(h + 1) * head_dim] = p @ vv
    return out


def test_q8_attention_against_f64_brute_force():
    heads, kvh, head_dim, cached = 16, 8, 128, 37
    kvw = kvh * head_dim
    k = normal(cached * kvw, 3, 1).reshape(cached, kvw)
    v = normal(cached * kvw, 3, 2).reshape(cached, kvw)
    q = normal(heads * head_dim, 3, 3)
    ks, kc = _q8_planes(k)
    vs, vc = _q8_planes(v)
    kd = o.dequantize_rows(o.Q8, ks, kc, cached, kvw).astype(np.float64)
    vd = o.dequantize_rows(o.Q8, vs, vc, cached, kvw).astype(np.float64)
    expected = _attention_f64(q, kd, vd, heads, kvh, head_dim)
    actual = o.decode_attention_q8(q, ks, kc, vs, vc, cached, heads, kvh, head_dim)
    assert np.all(np.abs(actual - expected) <= 1e-5 * (np.abs(expected) + 1))


def test_q8_attention_identical_keys_average_values():
    # Closed form: equal scores give the mean of the (dequantized) values.
    heads, kvh, head_dim, cached = 4, 2, 64, 9
    kvw = kvh * head_dim
    k = np.tile(normal(kvw, 5, 1), (cached, 1))
    v = normal(cached * kvw, 5, 2).reshape(cached, kvw)
    q = normal(heads * head_dim, 5, 3)
    ks, kc = _q8_planes(k)
    vs, vc = _q8_planes(v)
    vd = o.dequantize_rows(o.Q8, vs, vc, cached, kvw).astype(np.float64)
    actual = o.decode_attention_q8(q, ks, kc, vs, vc, cached, heads, kvh, head_dim)
    for h in range(heads):
        g = h // 2
        assert np.allclose(actual[h * head_dim:(h + 1) * head_dim], vd[:, g * head_dim:(g + 1) * head_dim].mean(0),
                           rtol=1e-5, atol=1e-6)


def test_decode_attention_mirror_symmetry():
    # kernels.zig:1119-1138
    out = o.decode_attention(np.array([1, 0, 0, 1], np.float32), np.array([1, 0, 0, 1], np.float32),
                             np.array([1, 1, 3, 3], np.float32), 2, 2, 1, 2)
    assert out[0] < 2.0 and out[2] > 2.0
    assert abs(out[0] + out[2] - 4.0) <= 1e-5 and abs(out[1] + out[3] - 4.0) <= 1e-5


def test_q8_attention_rejects_bad_shapes():
    lib = o.lib()
    z = np.zeros(1024, np.uint8)
    f = np.zeros(256, np.float32)
    # head_dim not a multiple of 64, heads not a multiple of kv_heads
    assert lib.qwref_decode_attention_step_q8(f.ctypes.data, f.ctypes.data, z.ctypes.data, z.ctypes.data,
                                              z.ctypes.data, z.ctypes.data, 1, 2, 1, 32) == -7
    assert lib.qwref_decode_attention_step_q8(f.ctypes.data, f.ctypes.data, z.ctypes.data, z.ctypes.data,
                                              z.ctypes.data, z.ctypes.data, 1, 3, 2, 64) == -7


# ---------------------------------------------------------------- glue
def test_math_known_answers():
    # math.zig:174-214
    assert abs(o.silu(0.0)) <= 1e-7
    assert abs(o.silu(1.0) - 0.7310586) <= 1e-6
    assert abs(o.silu(-1.0) + 0.26894143) <= 1e-6
    assert abs(o.silu(30.0) - 30.0) <= 1e-3 and abs(o.silu(-30.0)) <= 1e-9
    row = o.softmax([1.0, 2.0, 3.0])
    assert abs(row.sum() - 1.0) <= 1e-6
    assert np.allclose(row, [0.09003057, 0.24472848, 0.66524096], atol=1e-6)
    ext = o.softmax([1000.0, -1000.0, 0.0])
    assert abs(ext[0] - 1.0) <= 1e-6 and ext[1] == 0.0
    r = o.rms_norm([3.0, 4.0], np.ones(2, np.float32), 2, 0.0)
    assert abs((r[0] ** 2 + r[1] ** 2) / 2 - 1.0) <= 1e-6
    assert np.all(o.rms_norm([0.0, 0.0, 0.0], np.ones(3, np.float32), 3, 1e-6) == 0.0)
    gate = np.array([0.0, 1.0, -1.0], np.float32)
    up = np.array([1.0, 2.0, 3.0], np.float32)
    out = o.silu_mul(gate, up)
    assert abs(out[1] - o.silu(1.0) * 2) <= 1e-6 and abs(out[2] - o.silu(-1.0) * 3) <= 1e-6


def test_rms_norm_applies_each_weight_to_its_own_element():
    # math.zig:120-130: x * (1 / sqrt(mean(x^2) + eps)) * w. A row of +-1 has
    # mean square exactly 1, so with eps 0 the output is x_i * w_i exactly:
    # distinct weights catch a dropped, shifted or reversed weight index.
    x = np.array([1, -1, -1, 1, 1, 1, -1, 1], np.float32)
    w = np.arange(1, 9, dtype=np.float32) * np.float32(0.25) + np.float32(0.5)
    assert np.array_equal(o.rms_norm(x, w, 8, 0.0), x * w)
    # Several rows (tokens): each row normalized by its own statistics, the
    # same weight vector for every row; against float64.
    rows = normal(3 * 64, 5).reshape(3, 64) * np.array([[0.1], [1.0], [7.0]], np.float32)
    wv = 1.0 + 0.5 * normal(64, 6)
    got = o.rms_norm(rows.reshape(-1), wv, 64, 1e-6).reshape(3, 64)
    r64 = rows.astype(np.float64)
    want = r64 / np.sqrt(np.mean(r64 * r64, axis=1, keepdims=True) + 1e-6) * wv.astype(np.float64)
    assert np.allclose(got, want, rtol=2e-6, atol=0)


def test_rope_rotation_and_frequencies():
    # kernels.zig:1080-1117
    cos, sin = o.rope_tables(2, 1e6, 8)
    x = np.tile(np.array([1, 2, 3, 4], np.float32), 3)
    r = o.rope(x, [0, 1, 7], 1, 4, cos, sin).reshape(3, 4)
    assert np.allclose(r[0], [1, 2, 3, 4], atol=1e-6)
    assert np.allclose((r ** 2).sum(1), 30.0, atol=1e-4)
    assert abs(o.inverse_frequency(0, 128, 1e6) - 1.0) <= 1e-6
    assert abs(o.inverse_frequency(64, 128, 1e6) - 1e-6) <= 1e-12
    # rotate_half pairing (i, i + half): position 1 of head_dim 4 rotates
    # (x0, x2) by angle 1 and (x1, x3) by angle 1e-3.
    a0, a1 = 1.0, 1e6 ** (-0.5)
    expected = [1 * math.cos(a0) - 3 * math.sin(a0), 2 * math.cos(a1) - 4 * math.sin(a1),
                3 * math.cos(a0) + 1 * math.sin(a0), 4 * math.cos(a1) + 2 * math.sin(a1)]
    assert np.allclose(r[1], expected, atol=1e-5)


def test_argmax_lowest_index_of_equal_maxima():
    # harness.mjs:280-284: 1000 values, maxima at 333 and 777 -> 333.
    v = normal(1000, 0x5EED0014)
    v[777] = 4.0
    v[333] = 4.0
    assert o.argmax(v) == 333
    assert o.argmax(np.array([2.0, 2.0, 1.0], np.float32)) == 0


# ---------------------------------------------------------------- generator
def _mulberry32(state: int) -> int:
    v = state & 0xFFFFFFFF
    v = ((v ^ (v >> 15)) * (v | 1)) & 0xFFFFFFFF
    v = (v ^ ((v + (((v ^ (v >> 7)) * (v | 61)) & 0xFFFFFFFF)) & 0xFFFFFFFF)) & 0xFFFFFFFF
    return (v ^ (v >> 14)) & 0xFFFFFFFF


def test_mulberry32_matches_an_independent_restatement():
    # tests/gpu/reference.mjs:35-44 (state += 0x6d2b79f5 before each draw).
    for seed in (0, 1, 0x5EED0001):
        state = seed
        for n in range(1, 50):
            state = (state + 0x6D2B79F5) & 0xFFFFFFFF
            assert o.mulberry32_at(seed, n) == _mulberry32(state)


def test_synthetic_normals_match_box_muller_in_double():
    # Box-Muller with the platform's double log/cos/sqrt: the deterministic
    # restatement may differ from it by at most one f32 ulp.
    seed, stream, count = 4, 3, 20000
    base = o.stream_base(seed, stream)
    vals = o.normal(count, seed, stream)
    u1 = np.array([o.mulberry32_at(base, 2 * i + 1) for i in range(count)], np.float64)
    u2 = np.array([o.mulberry32_at(base, 2 * i + 2) for i in range(count)], np.float64)
    ref = (np.sqrt(-2 * np.log(1 - u1 / 2 ** 32)) * np.cos(2 * np.pi * u2 / 2 ** 32)).astype(np.float32)
    ulps = np.abs(vals.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
    assert ulps.max() <= 1
    assert np.mean(ulps == 0) > 0.99
    assert abs(vals.mean()) < 0.03 and abs(vals.std() - 1) < 0.03


# ---------------------------------------------------------------- decoder
TINY = dict(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=128, ffn=512, vocab=1000,
            max_positions=64, eps=1e-6, theta=1e6)


def _tiny_weights(seed, fmt=o.Q4):
    """The oracle's synthetic model, rebuilt through the public generator and
    quantizer (same stream ids), dequantized to f64."""
    c = TINY
    qw, kvw = c["heads"] * c["head_dim"], c["kv_heads"] * c["head_dim"]

    def mat(rows, cols, stream):
        values = o.normal(rows * cols, seed, stream, 0.02).reshape(rows, cols)
        if fmt == o.F32:
            return values.astype(np.float64)
        if fmt == o.F16:  # numpy's own f16 rounding, not the oracle's
            return values.astype(np.float16).astype(np.float64)
        s, d = o.quantize_rows(fmt, values)
        return o.dequantize_rows(fmt, s, d, rows, cols).astype(np.float64)

    w = {"embed": mat(c["vocab"], c["hidden"], 1), "lm_head": mat(c["vocab"], c["hidden"], 2), "layers": []}
    for layer in range(c["layers"]):
        b = 16 + 16 * layer
        w["layers"].append(dict(q=mat(qw, c["hidden"], b), k=mat(kvw, c["hidden"], b + 1),
                                v=mat(kvw, c["hidden"], b + 2), o=mat(c["hidden"], qw, b + 3),
                                gate=mat(c["ffn"], c["hidden"], b + 4), up=mat(c["ffn"], c["hidden"], b + 5),
                                down=mat(c["hidden"], c["ffn"], b + 6)))
    return w


def _random_norms(c, seed):
    """Norm weight vectors with distinct entries around 1 (a real checkpoint's
    learned norms are of this kind): per layer attention, q, k, ffn, and the
    final norm."""
    out = {"final": 1.0 + 0.5 * o.normal(c["hidden"], seed, 900)}
    for layer in range(c["layers"]):
        out[layer] = dict(attn=1.0 + 0.5 * o.normal(c["hidden"], seed, 901 + 8 * layer),
                          q=1.0 + 0.5 * o.normal(c["head_dim"], seed, 902 + 8 * layer),
                          k=1.0 + 0.5 * o.normal(c["head_dim"], seed, 903 + 8 * layer),
                          ffn=1.0 + 0.5 * o.normal(c["hidden"], seed, 904 + 8 * layer))
    return out


def _set_norms(dec, norms, layers):
    dec.set_vector(o.FINAL_NORM, 0, norms["final"])
    for layer in range(layers):
        n = norms[layer]
        dec.set_vector(o.ATTN_NORM, layer, n["attn"])
        dec.set_vector(o.Q_NORM, layer, n["q"])
        dec.set_vector(o.K_NORM, layer, n["k"])
        dec.set_vector(o.FFN_NORM, layer, n["ffn"])


def _forward_f64(w, tokens, c, norms=None, cache="q8"):
    """decoder.zig:133-287 in f64 (no rounding but the cache's): the
    composition the oracle must follow, written independently. With
    `norms`, every RMSNorm multiplies by its weight vector; `cache` "q8"
    stores quantizeRow(.q8) of each new key / value row, "f32" stores the f32
    rows."""
    hd, heads, kvh = c["head_dim"], c["heads"], c["kv_heads"]
    half = hd // 2
    inv = np.array([c["theta"] ** (-2 * i / hd) for i in range(half)])

    def weight(layer, name, size):
        if norms is None:
            return np.ones(size)
        return np.asarray(norms["final"] if layer is None else norms[layer][name], np.float64)

    def rms(x, wv, eps=c["eps"]):
        return x / np.sqrt(np.mean(x * x) + eps) * wv

    def rope(x, p):
        x = x.reshape(-1, hd).copy()
        a = p * inv
        lo, hi = x[:, :half].copy(), x[:, half:].copy()
        x[:, :half] = lo * np.cos(a) - hi * np.sin(a)
        x[:, half:] = hi * np.cos(a) + lo * np.sin(a)
        return x

    caches = [([], []) for _ in range(c["layers"])]
    logits = []
    for p, t in enumerate(tokens):
        h = w["embed"][t].copy()
        for layer, L in enumerate(w["layers"]):
            n = rms(h, weight(layer, "attn", c["hidden"]))
            wq, wk = weight(layer, "q", hd), weight(layer, "k", hd)
            q = rope(np.stack([rms(r, wq) for r in (L["q"] @ n).reshape(heads, hd)]).reshape(-1), p)
            k = rope(np.stack([rms(r, wk) for r in (L["k"] @ n).reshape(kvh, hd)]).reshape(-1), p).reshape(-1)
            v = (L["v"] @ n).reshape(kvh, hd)
            for store, row in ((caches[layer][0], k), (caches[layer][1], v.reshape(-1))):
                row32 = row.astype(np.float32).reshape(1, -1)
                if cache == "q8":
                    # appendCacheRow stores q8 of the f32 rows (decoder.zig:94-105).
                    rs, rd = o.quantize_rows(o.Q8, row32)
                    row32 = o.dequantize_rows(o.Q8, rs, rd, 1, row.size)
                store.append(row32.astype(np.float64).reshape(kvh, hd))
            K = np.stack(caches[layer][0])
            V = np.stack(caches[layer][1])
            att = np.zeros((heads, hd))
            for hh in range(heads):
                g = hh // (heads // kvh)
                sc = K[:, g] @ q[hh] / math.sqrt(hd)
                pr = np.exp(sc - sc.max())
                att[hh] = (pr / pr.sum()) @ V[:, g]
            h = h + L["o"] @ att.reshape(-1)
            n = rms(h, weight(layer, "ffn", c["hidden"]))
            g_ = L["gate"] @ n
            h = h + L["down"] @ (g_ / (1 + np.exp(-g_)) * (L["up"] @ n))
        logits.append(w["lm_head"] @ rms(h, weight(None, "final", c["hidden"])))
    return logits


@pytest.mark.parametrize("fmt,cache,with_norms", [
    (o.Q4, o.CACHE_Q8, False),
    (o.Q4, o.CACHE_Q8, True),
    (o.Q8, o.CACHE_Q8, True),
    (o.Q5, o.CACHE_F32, True),
    (o.Q4, o.CACHE_F32, False),
    (o.F16, o.CACHE_Q8, True),
    (o.F32, o.CACHE_F32, True),
])
def test_decoder_composition_against_f64_restatement(fmt, cache, with_norms):
    seed = 9
    w = _tiny_weights(seed, fmt)
    norms = _random_norms(TINY, 31) if with_norms else None
    tokens = [5, 977, 123, 42]
    expected = _forward_f64(w, tokens, TINY, norms, "q8" if cache == o.CACHE_Q8 else "f32")
    dec = o.Decoder(seed, 1, fmt, cache, **TINY)
    try:
        if norms is not None:
            _set_norms(dec, norms, TINY["layers"])
        for i, t in enumerate(tokens):
            dec.forward(0, t, True)
            got = dec.logits(0)
            # Both sides store the same cache; what remains is f32 rounding
            # (and, rarely, a q8 code that an f32-vs-f64 difference flips).
            assert np.max(np.abs(got - expected[i])) < 2e-4 * max(1.0, np.abs(expected[i]).max()), i
        assert dec.position(0) == len(tokens)
    finally:
        dec.close()


def test_decoder_norm_weights_change_the_result():
    # A norm vector that is set must reach the step: each of the five kinds,
    # changed alone, changes the logits (a dropped weight would not).
    seed = 9
    # (A prefilled cache: with one position the softmax weight is 1 whatever
    # the query, so the q norm could not show.)
    base = o.Decoder(seed, 1, **TINY)
    base.prefill_random(0, 6)
    base.forward(0, 5, True)
    ref = base.logits(0)
    base.close()
    for kind, size in ((o.ATTN_NORM, TINY["hidden"]), (o.Q_NORM, TINY["head_dim"]), (o.K_NORM, TINY["head_dim"]),
                       (o.FFN_NORM, TINY["hidden"]), (o.FINAL_NORM, TINY["hidden"])):
        dec = o.Decoder(seed, 1, **TINY)
        try:
            dec.set_vector(kind, 1, 1.0 + 0.5 * o.normal(size, 3, kind))
            dec.prefill_random(0, 6)
            dec.forward(0, 5, True)
            assert np.max(np.abs(dec.logits(0) - ref)) > 1e-3, kind
            with pytest.raises(ValueError):
                dec.set_vector(kind, 0, np.ones(size + 1, np.float32))
        finally:
            dec.close()


def test_decoder_step_argmax_and_position_limit():
    dec = o.Decoder(3, 1, **{**TINY, "max_positions": 3})
    try:
        t = 7
        for _ in range(3):
            nxt = dec.step(0, t)
            assert nxt == o.argmax(dec.logits(0))
            t = nxt
        with pytest.raises(ValueError):
            dec.step(0, t)  # decoder.zig:142 PositionExceeded
    finally:
        dec.close()


def test_decoder_cache_row_reads_the_prefilled_rows():
    # decoder.zig:85-105: a prefilled q8 row is quantizeRow(.q8) of the
    # generator's values (stream 0x10000 + 0x100 seq + 2 layer + kv); the f32
    # cache keeps the values themselves (decoder.zig:77-83).
    cfg = dict(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=128, ffn=512, vocab=1000,
               max_positions=16, eps=1e-6, theta=1e6)
    kvw = cfg["kv_heads"] * cfg["head_dim"]
    for cache in (o.CACHE_Q8, o.CACHE_F32):
        d = o.Decoder(7, 2, o.Q4, cache, **cfg)
        try:
            d.prefill_random(1, 5)
            for layer in range(2):
                rows = [o.normal(5 * kvw, 7, 0x10000 + 0x100 * 1 + 2 * layer + kv).reshape(5, kvw) for kv in (0, 1)]
                for p in (0, 4):
                    got = d.cache_row(1, layer, p)
                    if cache == o.CACHE_F32:
                        want = rows[0][p].tobytes() + rows[1][p].tobytes()
                    else:
                        want = b"".join(s.tobytes() + c.tobytes()
                                        for s, c in (o.quantize_rows(o.Q8, r[p:p + 1]) for r in rows))
                    assert got == want, (cache, layer, p)
            with pytest.raises(ValueError):
                d.cache_row(2, 0, 0)
        finally:
            d.close()


def test_decoder_set_cache_row_and_position():
    # The checker's plumbing (teacher forcing on another implementation's
    # rows): rows stored through set_cache_row read back as they were, a
    # decoder given another's rows and position then steps exactly as that
    # decoder does, and a planted wrong row changes the next logits.
    cfg = dict(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=128, ffn=512, vocab=1000,
               max_positions=16, eps=1e-6, theta=1e6)
    for cache in (o.CACHE_Q8, o.CACHE_F32):
        a = o.Decoder(3, 1, o.Q4, cache, **cfg)
        b = o.Decoder(3, 1, o.Q4, cache, **cfg)
        try:
            a.prefill_random(0, 5)
            a.forward(0, 11, False)
            for layer in range(2):
                for p in range(6):
                    b.set_cache_row(0, layer, p, a.cache_row(0, layer, p))
            b.set_position(0, 6)
            assert a.cache_hash(0) == b.cache_hash(0) and b.position(0) == 6
            a.forward(0, 7)
            b.forward(0, 7)
            assert np.array_equal(a.logits(0), b.logits(0))
            row = bytearray(a.cache_row(0, 1, 3))
            row[len(row) // 2 - 1] ^= 0x40            # one code (q8) / one value byte (f32)
            b.set_position(0, 7)
            b.set_cache_row(0, 1, 3, bytes(row))
            assert b.cache_row(0, 1, 3) == bytes(row)
            a.forward(0, 9)
            b.forward(0, 9)
            assert not np.array_equal(a.logits(0), b.logits(0))
            with pytest.raises(ValueError):
                b.set_cache_row(0, 0, 0, bytes(row[:-1]))
            with pytest.raises(ValueError):
                b.set_position(0, 17)
        finally:
            a.close()
            b.close()
