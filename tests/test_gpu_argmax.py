"""decoder.zig:290-301 argmaxLogits on the device (qwh_argmax_rows, the
decoder step's argmax kernels) against the oracle's restatement
(oracle/qwref.c qwref_argmax), on the reference harness's tie case and on
ties, NaNs and infinities placed around the kernels' 4096-logit blocks."""
import numpy as np
import pytest

from oracle import oracle as o
from util import normal

pytestmark = pytest.mark.gpu


def device_argmax(ctx, rows):
    rows = np.ascontiguousarray(rows, np.float32)
    n, count = rows.shape
    x = ctx.to_device(rows.reshape(-1))
    ids = ctx.buffer(4 * n)
    try:
        ctx.argmax_rows(x.ptr, n, count, ids.ptr)
        return ids.download(np.uint32).tolist()
    finally:
        x.free()
        ids.free()


def test_harness_tie_case(ctx):
    # harness.mjs:280-284: 1000 values, equal maxima at 333 and 777 -> 333.
    v = np.zeros((1, 1000), np.float32)
    v[0, 777] = 4.0
    v[0, 333] = 4.0
    assert device_argmax(ctx, v) == [333] == [o.argmax(v[0])]


def test_ties_nans_and_infinities(ctx):
    vocab = 151936
    rows = normal(12 * vocab, 41).reshape(12, vocab)
    rows[0, [1023, 1024, 4096, 9000]] = 9.0    # a tie across a block boundary: the first
    rows[1, [150000, 70000]] = 9.0              # a later block holds the lower index
    rows[2, 0] = np.nan                          # NaN first: the reference keeps index 0
    rows[3, 5] = np.nan                          # NaN elsewhere is never the maximum
    rows[3, 6] = 9.0
    rows[4, :] = -np.inf                         # nothing above -inf: index 0
    rows[5, :] = np.nan                          # all NaN: index 0
    rows[6, 100] = np.inf                        # +inf wins; a second +inf later loses the tie
    rows[6, 200] = np.inf
    rows[7, :] = 1.0                             # all equal: index 0
    rows[8, vocab - 1] = 9.0                     # the last index
    rows[9, 0] = -np.inf                         # first value -inf, the rest finite
    rows[10, :] = -3.4028235e38                  # every value -FLT_MAX: index 0
    rows[11, 1::2] = np.nan                      # NaNs between finite values
    got = device_argmax(ctx, rows)
    want = [o.argmax(r) for r in rows]
    assert got == want, (got, want)


@pytest.mark.parametrize("count", [1, 2, 3, 1000, 1023, 1024, 1025, 1027, 4095, 4096, 4097])
def test_row_lengths(ctx, count):
    rows = normal(3 * count, 42 + count).reshape(3, count)
    assert device_argmax(ctx, rows) == [o.argmax(r) for r in rows]


@pytest.mark.parametrize("offset", [1, 2, 3])
def test_rows_not_16_byte_aligned(ctx, offset):
    # Logits that start 4, 8 or 12 bytes past a 16-byte boundary (a slice of
    # a larger buffer): every row and block then starts unaligned, and the
    # kernel reads them without 16-byte loads.
    count = 4099
    rows = normal(2 * count, 43 + offset).reshape(2, count)
    rows[1, 2050] = 9.0
    flat = np.concatenate([np.zeros(offset, np.float32), rows.reshape(-1)])
    x = ctx.to_device(flat)
    ids = ctx.buffer(8)
    try:
        ctx.argmax_rows(x.ptr + 4 * offset, 2, count, ids.ptr)
        got = ids.download(np.uint32).tolist()
    finally:
        x.free()
        ids.free()
    assert got == [o.argmax(r) for r in rows]
