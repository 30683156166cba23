"""GPU parity of the f32-cache decode attention (kernels.zig:572-627
decodeAttentionStep, the reference's default cache) against the oracle."""
import os

import numpy as np
import pytest

from oracle import oracle as o
from util import assert_close, lcg_values

pytestmark = pytest.mark.gpu
o.set_threads(min(16, os.cpu_count() or 1))


def run_f32(ctx, q, keys, values, cached, heads, kvh, hd, batch=1, stride=0):
    kb = ctx.to_device(np.ascontiguousarray(keys, np.float32))
    vb = ctx.to_device(np.ascontiguousarray(values, np.float32))
    qb = ctx.to_device(np.ascontiguousarray(q, np.float32))
    ob = ctx.buffer(batch * heads * hd * 4)
    ctx.decode_attention_f32(ob.ptr, qb.ptr, kb.ptr, vb.ptr, cached, heads, kvh, hd, batch, stride)
    out = ob.download(np.float32)
    for b in (kb, vb, qb, ob):
        b.free()
    return out


def test_reference_lcg_case(ctx):
    # kernels.zig:769-836 inputs: the f32 attention the q8 test compares with.
    hd, kvh, heads, cached = 64, 2, 4, 5
    kvw = kvh * hd
    keys, state = lcg_values(cached * kvw, 7, 200.0)
    values, state = lcg_values(cached * kvw, state, 400.0)
    query, state = lcg_values(heads * hd, state, 500.0)
    expected = o.decode_attention(query, keys, values, cached, heads, kvh, hd)
    actual = run_f32(ctx, query, keys, values, cached, heads, kvh, hd)
    assert_close(actual, expected, rtol=1e-4, atol_rms=1e-4, what="reference LCG case, f32 cache")


@pytest.mark.parametrize("ctx_len", [512, 4096, 8192])
@pytest.mark.parametrize("batch", [1, 8])
def test_config4_shapes_f32_cache(ctx, ctx_len, batch):
    heads, kvh, hd = 16, 8, 128
    kvw = kvh * hd
    keys = [o.normal(ctx_len * kvw, 3, 10 * b) for b in range(batch)]
    values = [o.normal(ctx_len * kvw, 3, 10 * b + 1) for b in range(batch)]
    q = o.normal(batch * heads * hd, 3, 999)
    expected = np.concatenate([o.decode_attention(q[b * heads * hd:(b + 1) * heads * hd], keys[b], values[b], ctx_len,
                                                  heads, kvh, hd) for b in range(batch)])
    actual = run_f32(ctx, q, np.concatenate(keys), np.concatenate(values), ctx_len, heads, kvh, hd, batch,
                     keys[0].nbytes)
    assert_close(actual, expected, what=f"f32 cache ctx {ctx_len} batch {batch}")


@pytest.mark.parametrize("cached,hd,heads,kvh", [(1, 128, 16, 8), (129, 64, 8, 4), (300, 256, 4, 2),
                                                 (77, 128, 8, 8), (513, 128, 16, 2), (4099, 128, 16, 8)])
def test_f32_attention_edge_shapes(ctx, cached, hd, heads, kvh):
    kvw = kvh * hd
    keys = o.normal(cached * kvw, 14, 0)
    values = o.normal(cached * kvw, 14, 1)
    q = o.normal(heads * hd, 14, 5)
    expected = o.decode_attention(q, keys, values, cached, heads, kvh, hd)
    actual = run_f32(ctx, q, keys, values, cached, heads, kvh, hd)
    assert_close(actual, expected, what=f"f32 attention cached {cached} hd {hd} {heads}/{kvh}")


def test_f32_attention_reads_only_the_cached_positions(ctx):
    # kernels.zig:1119-1138: two query heads over one kv head of two
    # dimensions and two cached rows; head 0 leans to value 0, head 1 to
    # value 1, and the two mirror each other. The buffers hold four more rows
    # of NaN past the cached two: reading any of them would show in the
    # output.
    q = np.array([1.0, 0.0, 0.0, 1.0], np.float32)
    keys = np.full(12, np.nan, np.float32)
    values = np.full(12, np.nan, np.float32)
    keys[:4] = [1.0, 0.0, 0.0, 1.0]
    values[:4] = [1.0, 1.0, 3.0, 3.0]
    out = run_f32(ctx, q, keys, values, 2, 2, 1, 2)
    assert np.all(np.isfinite(out))
    assert out[0] < 2.0 and out[2] > 2.0
    assert abs(out[0] + out[2] - 4.0) <= 1e-5 and abs(out[1] + out[3] - 4.0) <= 1e-5
    expected = o.decode_attention(q, keys[:4], values[:4], 2, 2, 1, 2)
    assert_close(out, expected, rtol=1e-5, atol_rms=1e-6, what="two cached rows")


def test_f32_identical_keys_give_the_mean_of_values(ctx):
    # Equal scores: softmax weights 1/cached, the output the mean of V.
    heads, kvh, hd, cached = 16, 8, 128, 333
    kvw = kvh * hd
    keys = np.tile(o.normal(kvw, 13, 1), cached)
    values = o.normal(cached * kvw, 13, 2).reshape(cached, kvw)
    q = o.normal(heads * hd, 13, 3)
    actual = run_f32(ctx, q, keys, values.reshape(-1), cached, heads, kvh, hd).reshape(heads, hd)
    mean = values.astype(np.float64).mean(axis=0).reshape(kvh, hd)
    for h in range(heads):
        assert np.allclose(actual[h], mean[h // (heads // kvh)], atol=1e-5), h


@pytest.mark.parametrize("cached,hd,heads,kvh,batch", [(300, 192, 6, 2, 1), (129, 96, 3, 1, 1), (77, 40, 10, 2, 1),
                                                       (513, 1024, 2, 1, 1), (200, 320, 9, 3, 2)])
def test_f32_attention_any_head_shape(ctx, cached, hd, heads, kvh, batch):
    # kernels.zig:583-593 takes any head_dim and any heads / kv_heads ratio:
    # these run the one-workgroup-per-head kernel.
    kvw = kvh * hd
    keys = [o.normal(cached * kvw, 23, 10 * b) for b in range(batch)]
    values = [o.normal(cached * kvw, 23, 10 * b + 1) for b in range(batch)]
    q = o.normal(batch * heads * hd, 23, 5)
    expected = np.concatenate([o.decode_attention(q[b * heads * hd:(b + 1) * heads * hd], keys[b], values[b], cached,
                                                  heads, kvh, hd) for b in range(batch)])
    stride = (keys[0].nbytes + 15) // 16 * 16
    pad = np.zeros((stride - keys[0].nbytes) // 4, np.float32)
    kcat = np.concatenate([np.concatenate([k, pad]) for k in keys])
    vcat = np.concatenate([np.concatenate([v, pad]) for v in values])
    actual = run_f32(ctx, q, kcat, vcat, cached, heads, kvh, hd, batch, stride if batch > 1 else 0)
    assert_close(actual, expected, what=f"f32 attention cached {cached} hd {hd} {heads}/{kvh} batch {batch}")
