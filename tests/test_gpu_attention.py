"""GPU parity of the q8 key/value cache decode attention
(kernels.zig:697-767 decodeAttentionStepQ8) against the oracle."""
import os

import numpy as np
import pytest

import qwenscriber_amd as qa
from oracle import oracle as o
from util import assert_close, lcg_values

pytestmark = pytest.mark.gpu
o.set_threads(min(16, os.cpu_count() or 1))


def make_cache(cached, kvw, seed, stream):
    k = o.normal(cached * kvw, seed, stream).reshape(cached, kvw)
    v = o.normal(cached * kvw, seed, stream + 1).reshape(cached, kvw)
    ks, kc = o.quantize_rows(o.Q8, k)
    vs, vc = o.quantize_rows(o.Q8, v)
    return ks, kc, vs, vc


def run_attention(ctx, q, planes, cached, heads, kvh, hd, batch=1, scale_stride=0, code_stride=0):
    bufs = [ctx.to_device(np.ascontiguousarray(p)) for p in planes]
    qb = ctx.to_device(np.ascontiguousarray(q, np.float32))
    ob = ctx.buffer(batch * heads * hd * 4)
    ctx.decode_attention_q8(ob.ptr, qb.ptr, *[b.ptr for b in bufs], cached, heads, kvh, hd, batch,
                            scale_stride, code_stride)
    out = ob.download(np.float32)
    for b in bufs + [qb, ob]:
        b.free()
    return out


def test_harness_decode_attention_case(ctx):
    # harness.mjs:289-323, :537-571: heads 4, kv heads 2, head_dim 128, 5
    # positions, seeds 0x5eed0016 / 17 / 18.
    heads, kvh, hd, cached = 4, 2, 128, 5
    q = o.normal(heads * hd, 0x5EED0016)
    k = o.normal(cached * kvh * hd, 0x5EED0017).reshape(cached, -1)
    v = o.normal(cached * kvh * hd, 0x5EED0018).reshape(cached, -1)
    ks, kc = o.quantize_rows(o.Q8, k)
    vs, vc = o.quantize_rows(o.Q8, v)
    expected = o.decode_attention_q8(q, ks, kc, vs, vc, cached, heads, kvh, hd)
    actual = run_attention(ctx, q, (ks, kc, vs, vc), cached, heads, kvh, hd)
    assert_close(actual, expected, rtol=1e-4, atol_rms=1e-4, what="harness decode_attention_q8")


def test_reference_lcg_case(ctx):
    # kernels.zig:769-836 inputs (head_dim 64, 4 heads over 2, 5 positions).
    hd, kvh, heads, cached = 64, 2, 4, 5
    kvw = kvh * hd
    keys, state = lcg_values(cached * kvw, 7, 200.0)
    values, state = lcg_values(cached * kvw, state, 400.0)
    query, state = lcg_values(heads * hd, state, 500.0)
    ks, kc = o.quantize_rows(o.Q8, keys.reshape(cached, kvw))
    vs, vc = o.quantize_rows(o.Q8, values.reshape(cached, kvw))
    expected = o.decode_attention_q8(query, ks, kc, vs, vc, cached, heads, kvh, hd)
    actual = run_attention(ctx, query, (ks, kc, vs, vc), cached, heads, kvh, hd)
    assert_close(actual, expected, what="reference LCG case")
    exact = o.decode_attention(query, keys, values, cached, heads, kvh, hd)
    assert np.all(np.abs(actual - exact) <= 0.05)


@pytest.mark.parametrize("ctx_len", [512, 2048, 4096, 8192])
@pytest.mark.parametrize("batch", [1, 8])
def test_config4_gqa_attention(ctx, ctx_len, batch):
    heads, kvh, hd = 16, 8, 128
    kvw = kvh * hd
    planes = [make_cache(ctx_len, kvw, 3, 10 * b) for b in range(batch)]
    q = o.normal(batch * heads * hd, 3, 999)
    expected = np.concatenate([o.decode_attention_q8(q[b * heads * hd:(b + 1) * heads * hd], *planes[b], ctx_len,
                                                     heads, kvh, hd) for b in range(batch)])
    stacked = [np.concatenate([planes[b][i] for b in range(batch)]) for i in range(4)]
    scale_stride = planes[0][0].nbytes
    code_stride = planes[0][1].nbytes
    actual = run_attention(ctx, q, stacked, ctx_len, heads, kvh, hd, batch, scale_stride, code_stride)
    assert_close(actual, expected, what=f"config 4 ctx {ctx_len} batch {batch}")


@pytest.mark.parametrize("cached,hd,heads,kvh", [(1, 128, 16, 8), (1000, 128, 16, 8), (129, 64, 8, 4),
                                                 (300, 256, 4, 2), (77, 128, 8, 8), (513, 128, 16, 4),
                                                 (200, 64, 4, 4), (150, 64, 8, 2), (400, 128, 16, 2),
                                                 (260, 256, 2, 2), (17, 128, 16, 8), (4099, 128, 16, 8)])
def test_attention_edge_shapes(ctx, cached, hd, heads, kvh):
    kvw = kvh * hd
    planes = make_cache(cached, kvw, 12, 0)
    q = o.normal(heads * hd, 12, 5)
    expected = o.decode_attention_q8(q, *planes, cached, heads, kvh, hd)
    actual = run_attention(ctx, q, planes, cached, heads, kvh, hd)
    assert_close(actual, expected, what=f"attention cached {cached} hd {hd} {heads}/{kvh}")


@pytest.mark.parametrize("cached,hd,heads,kvh", [(2, 64, 2, 1), (37, 128, 16, 8), (300, 64, 4, 4)])
def test_attention_reads_only_the_cached_positions(ctx, cached, hd, heads, kvh):
    # kernels.zig:1119-1138 for the q8 cache: rows past the cached count hold
    # NaN scales and codes 0xFF; the output must be finite and equal the
    # attention over the cached rows alone.
    kvw = kvh * hd
    extra = 40
    ks, kc, vs, vc = make_cache(cached, kvw, 17, cached)
    nan_scales = np.full(extra * kvw // 64, 0x7E00, np.uint16).view(np.uint8)
    planes = [np.concatenate([ks, nan_scales]), np.concatenate([kc, np.full(extra * kvw, 0xFF, np.uint8)]),
              np.concatenate([vs, nan_scales]), np.concatenate([vc, np.full(extra * kvw, 0xFF, np.uint8)])]
    q = o.normal(heads * hd, 17, 99)
    out = run_attention(ctx, q, planes, cached, heads, kvh, hd)
    assert np.all(np.isfinite(out))
    expected = o.decode_attention_q8(q, ks, kc, vs, vc, cached, heads, kvh, hd)
    assert_close(out, expected, what=f"{cached} cached rows before NaN rows")


def test_identical_keys_give_the_mean_of_values(ctx):
    heads, kvh, hd, cached = 16, 8, 128, 333
    kvw = kvh * hd
    k = np.tile(o.normal(kvw, 13, 1), (cached, 1))
    v = o.normal(cached * kvw, 13, 2).reshape(cached, kvw)
    ks, kc = o.quantize_rows(o.Q8, k)
    vs, vc = o.quantize_rows(o.Q8, v)
    vd = o.dequantize_rows(o.Q8, vs, vc, cached, kvw).astype(np.float64)
    q = o.normal(heads * hd, 13, 3)
    actual = run_attention(ctx, q, (ks, kc, vs, vc), cached, heads, kvh, hd).reshape(heads, hd)
    for h in range(heads):
        g = h // (heads // kvh)
        assert np.allclose(actual[h], vd[:, g * hd:(g + 1) * hd].mean(0), rtol=1e-5, atol=1e-5)


def test_attention_rejects_bad_shapes(ctx):
    buf = ctx.buffer(1 << 16)
    with pytest.raises(qa.QwhError) as err:
        ctx.decode_attention_q8(buf.ptr, buf.ptr, buf.ptr, buf.ptr, buf.ptr, buf.ptr, 4, 16, 8, 96)
    assert err.value.status == -7
    with pytest.raises(qa.QwhError) as err:
        ctx.decode_attention_q8(buf.ptr, buf.ptr, buf.ptr, buf.ptr, buf.ptr, buf.ptr, 0, 16, 8, 128)
    assert err.value.status == -7
    with pytest.raises(qa.QwhError) as err:
        ctx.decode_attention_q8(buf.ptr, buf.ptr, buf.ptr, buf.ptr, buf.ptr, buf.ptr, 4, 12, 8, 128)
    assert err.value.status == -7
    buf.free()


@pytest.mark.parametrize("cached,hd,heads,kvh,batch", [(300, 192, 6, 2, 1), (257, 320, 3, 1, 1), (1, 64, 12, 4, 1),
                                                       (600, 128, 24, 8, 1), (1030, 512, 4, 2, 1), (50, 1024, 2, 1, 1),
                                                       (700, 64, 10, 2, 1), (333, 192, 9, 3, 3)])
def test_attention_any_head_shape(ctx, cached, hd, heads, kvh, batch):
    # kernels.zig:712-716 takes any head_dim that is a multiple of 64 and any
    # heads / kv_heads ratio: these (head_dim 192 / 320 / 512 / 1024, ratios
    # 3 and 5) run the one-workgroup-per-head kernel.
    kvw = kvh * hd
    planes = [make_cache(cached, kvw, 21, 10 * b) for b in range(batch)]
    q = o.normal(batch * heads * hd, 21, 7)
    expected = np.concatenate([o.decode_attention_q8(q[b * heads * hd:(b + 1) * heads * hd], *planes[b], cached,
                                                     heads, kvh, hd) for b in range(batch)])
    stacked = [np.concatenate([planes[b][i] for b in range(batch)]) for i in range(4)]
    actual = run_attention(ctx, q, stacked, cached, heads, kvh, hd, batch, planes[0][0].nbytes, planes[0][1].nbytes)
    assert_close(actual, expected, what=f"attention cached {cached} hd {hd} {heads}/{kvh} batch {batch}")


def test_any_head_shape_identical_keys_give_the_mean_of_values(ctx):
    heads, kvh, hd, cached = 6, 2, 192, 300
    kvw = kvh * hd
    k = np.tile(o.normal(kvw, 22, 1), (cached, 1))
    v = o.normal(cached * kvw, 22, 2).reshape(cached, kvw)
    ks, kc = o.quantize_rows(o.Q8, k)
    vs, vc = o.quantize_rows(o.Q8, v)
    vd = o.dequantize_rows(o.Q8, vs, vc, cached, kvw).astype(np.float64)
    q = o.normal(heads * hd, 22, 3)
    actual = run_attention(ctx, q, (ks, kc, vs, vc), cached, heads, kvh, hd).reshape(heads, hd)
    for h in range(heads):
        g = h // (heads // kvh)
        assert np.allclose(actual[h], vd[:, g * hd:(g + 1) * hd].mean(0), rtol=1e-5, atol=1e-5)


def test_attention_rejects_heads_wider_than_built(ctx):
    buf = ctx.buffer(1 << 20)
    with pytest.raises(qa.QwhError) as err:
        ctx.decode_attention_q8(buf.ptr, buf.ptr, buf.ptr, buf.ptr, buf.ptr, buf.ptr, 4, 2, 1, 1088)
    assert err.value.status == -3
    buf.free()
