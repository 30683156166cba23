"""`.qw` shards in device memory: qwh_shard_load copies the payload once;
matrices borrowed from it (File.quantizedPlanes, container.zig:245-262) give
the oracle's linearQuantized result, element tensors come back bit exact."""
import os

import numpy as np
import pytest

import qwenscriber_amd as qa
from oracle import oracle as o
from oracle import shard as sh
from util import assert_close

pytestmark = pytest.mark.gpu
o.set_threads(min(16, os.cpu_count() or 1))

MATRICES = [  # (kind, layer, format, rows, cols)
    (sh.KIND_DECODER_Q, 1, o.Q4, 300, 1024),
    (sh.KIND_DECODER_K, 1, o.Q5, 130, 2048),
    (sh.KIND_DECODER_V, 1, o.Q8, 77, 512),
    (sh.KIND_DECODER_FFN_DOWN, 2, o.Q4, 64, 3072),
    (sh.KIND_DECODER_OUTPUT, 0, o.Q5, 1000, 1024),
]


def build_shard():
    tensors, weights = [], {}
    for i, (kind, layer, fmt, rows, cols) in enumerate(MATRICES):
        w = o.normal(rows * cols, 20, i, 0.02).reshape(rows, cols)
        scales, data = o.quantize_rows(fmt, w)
        weights[(kind, layer)] = (fmt, rows, cols, scales, data)
        tensors.append(dict(kind=kind, layer=layer, format=fmt, dims=(rows, cols),
                            payload=sh.quantized_payload(fmt, scales, data)))
    norm = o.normal(1024, 20, 99)
    tensors.append(dict(kind=sh.KIND_DECODER_FINAL_NORM, layer=0, format=sh.F32, dims=(1024,), payload=norm.tobytes()))
    return sh.build(tensors), weights, norm


def test_shard_matrices_and_tensors(ctx):
    data, weights, norm = build_shard()
    assert sh.parse(data)[0] == sh.OK
    shard = ctx.shard_load(data)
    handles = []
    try:
        for (kind, layer), (fmt, rows, cols, scales, wdata) in weights.items():
            m = ctx.shard_matrix(shard, kind, layer)
            handles.append(m)
            for tokens in (1, 3):
                x = o.normal(tokens * cols, 21, kind * 10 + tokens)
                xb = ctx.to_device(x)
                ob = ctx.buffer(tokens * rows * 4)
                ctx.linear(m, xb.ptr, cols, tokens, ob.ptr)
                actual = ob.download(np.float32).reshape(tokens, rows)
                expected = o.linear_quantized(fmt, scales, wdata, rows, cols, x, tokens)
                assert_close(actual, expected, what=f"shard kind {kind} layer {layer} tokens {tokens}")
                xb.free()
                ob.free()
        dev, entry = ctx.shard_tensor(shard, sh.KIND_DECODER_FINAL_NORM, 0)
        assert entry.format == sh.F32 and entry.dims[0] == 1024
        back = np.empty(1024, np.float32)
        ctx._check(ctx.lib.qwh_download(ctx.handle, back.ctypes.data, dev, back.nbytes))
        assert back.tobytes() == norm.tobytes()
        # Absent tensors, element tensors as matrices, release while borrowed.
        with pytest.raises(qa.QwhError) as err:
            ctx.shard_matrix(shard, sh.KIND_DECODER_Q, 5)
        assert err.value.status == sh.NOT_FOUND
        with pytest.raises(qa.QwhError) as err:
            ctx.shard_matrix(shard, sh.KIND_DECODER_FINAL_NORM, 0)
        assert err.value.status == sh.NOT_FOUND
        with pytest.raises(qa.QwhError) as err:
            ctx.shard_release(shard)
        assert err.value.status == -8
    finally:
        for m in handles:
            ctx.matrix_release(m)
    ctx.shard_release(shard)


def test_shard_load_rejects_corrupt_bytes(ctx):
    data, _, _ = build_shard()
    bad = bytearray(data)
    bad[0] = ord("X")
    with pytest.raises(qa.QwhError) as err:
        ctx.shard_load(bytes(bad))
    assert err.value.status == sh.BAD_MAGIC
