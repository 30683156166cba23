"""The allocation-free q8 decode attention (qwh_decode_attention_q8_noalloc)
against the allocating entry point (qwh_decode_attention_q8) on the same
inputs: identical results on two calls in a row, the second smaller than the
first (the static scratch keeps the first call's records), and a refusal of
inputs whose records exceed the static scratch."""
import ctypes
import os

import numpy as np
import pytest

import qwenscriber_amd as qa
from oracle import oracle as o
from util import assert_close

pytestmark = pytest.mark.gpu
o.set_threads(min(16, os.cpu_count() or 1))


def planes(batch, cached, kvw, seed):
    out = []
    for b in range(batch):
        k = o.normal(cached * kvw, seed, 10 * b).reshape(cached, kvw)
        v = o.normal(cached * kvw, seed, 10 * b + 1).reshape(cached, kvw)
        out.append(o.quantize_rows(o.Q8, k) + o.quantize_rows(o.Q8, v))
    return [np.concatenate([p[i] for p in out]) for i in range(4)], out


def call(ctx, fn, q, stacked, cached, heads, kvh, hd, batch, scale_stride, code_stride):
    bufs = [ctx.to_device(np.ascontiguousarray(p)) for p in stacked]
    qb = ctx.to_device(q)
    ob = ctx.buffer(batch * heads * hd * 4)
    ctx._check(fn(ctx.handle, ob.ptr, qb.ptr, *[b.ptr for b in bufs], cached, heads, kvh, hd, batch, scale_stride,
                  code_stride))
    out = ob.download(np.float32)
    for b in bufs + [qb, ob]:
        b.free()
    return out


@pytest.mark.parametrize("first,second", [((8, 4096, 16, 8, 128), (2, 300, 16, 8, 128)),
                                          ((1, 8192, 16, 8, 128), (3, 77, 8, 2, 64))])
def test_noalloc_matches_allocating_entry_point(ctx, first, second):
    for batch, cached, heads, kvh, hd in (first, second):
        kvw = kvh * hd
        stacked, per_seq = planes(batch, cached, kvw, 21)
        q = o.normal(batch * heads * hd, 21, 999)
        strides = (per_seq[0][0].nbytes, per_seq[0][1].nbytes)
        free = call(ctx, ctx.lib.qwh_decode_attention_q8_noalloc, q, stacked, cached, heads, kvh, hd, batch, *strides)
        alloc = call(ctx, ctx.lib.qwh_decode_attention_q8, q, stacked, cached, heads, kvh, hd, batch, *strides)
        # The same kernels in the same order: bit-identical results.
        assert np.array_equal(free, alloc), (batch, cached)
        expected = np.concatenate([o.decode_attention_q8(q[b * heads * hd:(b + 1) * heads * hd], *per_seq[b], cached,
                                                         heads, kvh, hd) for b in range(batch)])
        assert_close(free, expected, what=f"no-alloc attention batch {batch} cached {cached}")


def test_noalloc_refuses_records_beyond_its_scratch(ctx):
    # 1024 sequences x 8 kv heads of one range each: 8192 records of
    # 2 x 128 + 8 floats, above the 8 MiB static scratch. Refused before any
    # launch; the buffers still cover every row the call names.
    batch, cached, heads, kvh, hd = 1024, 1, 16, 8, 128
    kvw = kvh * hd
    scales = ctx.buffer(batch * (kvw // 64) * 2)
    codes = ctx.buffer(batch * kvw)
    q = ctx.buffer(batch * heads * hd * 4)
    out = ctx.buffer(batch * heads * hd * 4)
    with pytest.raises(qa.QwhError, match="limit_exceeded"):
        ctx._check(ctx.lib.qwh_decode_attention_q8_noalloc(ctx.handle, out.ptr, q.ptr, scales.ptr, codes.ptr,
                                                           scales.ptr, codes.ptr, cached, heads, kvh, hd, batch,
                                                           (kvw // 64) * 2, kvw))
    for b in (scales, codes, q, out):
        b.free()
