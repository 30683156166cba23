"""`.qw` shard parsing (container.zig) on the host: the library's
qwh_shard_validate / _find / _verify_checksum and the oracle's restatement,
each against the cases container.zig's own tests hold (:450-549) and the
remaining rules of File.parse. No device is needed."""
import struct

import numpy as np
import pytest

import qwenscriber_amd as qa
from oracle import oracle as o
from oracle import shard as sh


def one_tensor_shard(payload: bytes, fmt: int, rows: int, cols: int) -> bytes:
    # container.zig:553-582 testShard: one audio.conv1.weight tensor.
    return sh.build([dict(kind=sh.KIND_AUDIO_CONV1_WEIGHT, layer=0, format=fmt, dims=(rows, cols), payload=payload)])


def statuses(data: bytes):
    lib_status, _ = qa.shard_validate(data)
    oracle_status, _ = sh.parse(data)
    return lib_status, oracle_status


def test_minimal_shard_parses_and_exposes_its_tensor():
    # container.zig:450-472: q4 64 x 64 (64 groups), one nonzero byte in each
    # plane so swapped planes would show.
    _, data_off, total = sh.quantized_len(o.Q4, 64, 64)
    payload = bytearray(total)
    payload[data_off] = 0x0F
    payload[0] = 0x3C
    data = one_tensor_shard(bytes(payload), o.Q4, 64, 64)
    assert qa.shard_validate(data) == (0, 1)
    assert sh.parse(data)[0] == sh.OK
    status, entry = qa.shard_find(data, sh.KIND_AUDIO_CONV1_WEIGHT, 0)
    assert status == 0 and entry.format == o.Q4 and list(entry.dims[:2]) == [64, 64] and entry.rank == 2
    payload_offset = struct.unpack_from("<I", data, 16)[0]
    assert data[payload_offset + entry.offset_bytes + data_off] == 0x0F
    assert data[payload_offset + entry.offset_bytes] == 0x3C
    assert qa.shard_verify_checksum(data) == 0 and sh.verify_checksum(data) == sh.OK
    corrupted = bytearray(data)
    corrupted[-1] ^= 0xFF
    assert qa.shard_validate(bytes(corrupted))[0] == 0
    assert qa.shard_verify_checksum(bytes(corrupted)) == sh.CHECKSUM_MISMATCH
    assert sh.verify_checksum(bytes(corrupted)) == sh.CHECKSUM_MISMATCH


def test_lookup_is_by_kind_and_layer():
    # container.zig:474-486: q8 64 x 64 is 64 * (2 + 64) = 4224 bytes.
    data = one_tensor_shard(bytes(4224), o.Q8, 64, 64)
    assert qa.shard_find(data, sh.KIND_AUDIO_CONV1_WEIGHT, 0)[0] == 0
    assert qa.shard_find(data, sh.KIND_AUDIO_CONV1_WEIGHT, 1)[0] == sh.NOT_FOUND
    assert qa.shard_find(data, sh.KIND_AUDIO_CONV2_WEIGHT, 0)[0] == sh.NOT_FOUND
    _, entries = sh.parse(data)
    assert sh.find(entries, sh.KIND_AUDIO_CONV1_WEIGHT, 0) is not None
    assert sh.find(entries, sh.KIND_AUDIO_CONV1_WEIGHT, 1) is None


@pytest.mark.parametrize("offset,value,expected", [
    (0, ord("X"), sh.BAD_MAGIC),   # container.zig:494-497
    (8, 99, sh.BAD_VERSION),
    (24, 3, sh.TRUNCATED),          # tensor count disagrees with the index length
    (12, 0, sh.TRUNCATED),
    (16, 64, sh.TRUNCATED),         # payload offset overlaps the index
    (16, 300, sh.TRUNCATED),        # payload offset not a multiple of 256
])
def test_corrupt_headers_are_rejected(offset, value, expected):
    good = one_tensor_shard(bytes(4224), o.Q8, 64, 64)
    corrupt = bytearray(good)
    struct.pack_into("<I", corrupt, offset, value)
    assert statuses(bytes(corrupt)) == (expected, expected)


def test_truncated_buffers_are_rejected():
    good = one_tensor_shard(bytes(4224), o.Q8, 64, 64)
    for cut in (good[:16], good[:-1], good[:40]):
        assert statuses(cut) == (sh.TRUNCATED, sh.TRUNCATED)


def test_length_that_disagrees_with_shape_is_rejected():
    # container.zig:510-519: len_bytes at offset 32 of the first entry.
    good = one_tensor_shard(bytes(4224), o.Q8, 64, 64)
    corrupt = bytearray(good)
    struct.pack_into("<Q", corrupt, sh.HEADER_BYTES + 32, 8)
    assert statuses(bytes(corrupt)) == (sh.SHAPE_MISMATCH, sh.SHAPE_MISMATCH)


def entry_shard(entries, payload_len, count=None):
    """A shard whose index is written as given (no sorting or checks)."""
    index = b"".join(struct.pack("<HHBBH4I2Q", *e) for e in entries)
    count = len(entries) if count is None else count
    payload_offset = sh._up(sh.HEADER_BYTES + len(index), sh.PAYLOAD_ALIGN)
    payload = bytes(payload_len)
    header = sh.MAGIC + struct.pack("<6I", 1, len(index), payload_offset, payload_len, count, sh.checksum(payload))
    return header + index + bytes(payload_offset - sh.HEADER_BYTES - len(index)) + payload


F32_ENTRY = lambda kind, layer, n, off: (kind, layer, sh.F32, 1, 0, n, 1, 1, 1, off, 4 * n)


@pytest.mark.parametrize("entries,payload_len,expected", [
    # Sorted by (layer, kind): a later entry with a smaller key.
    ([F32_ENTRY(5, 1, 4, 0), F32_ENTRY(4, 1, 4, 16)], 32, sh.INVALID_ARGUMENT),
    ([F32_ENTRY(5, 2, 4, 0), F32_ENTRY(9, 1, 4, 16)], 32, sh.INVALID_ARGUMENT),
    # The same key twice.
    ([F32_ENTRY(5, 1, 4, 0), F32_ENTRY(5, 1, 4, 16)], 32, sh.INVALID_ARGUMENT),
    # Overlapping ranges.
    ([F32_ENTRY(5, 1, 8, 0), F32_ENTRY(6, 1, 4, 16)], 48, sh.INVALID_ARGUMENT),
    # A range past the payload.
    ([F32_ENTRY(5, 1, 8, 16)], 32, sh.TRUNCATED),
    # An element tensor at an offset that is not a multiple of 16.
    ([F32_ENTRY(5, 1, 2, 8)], 32, sh.INVALID_ARGUMENT),
    # A quantized tensor at such an offset: its planes no longer start at it.
    ([(1, 0, o.Q8, 2, 0, 1, 64, 1, 1, 8, 80)], 160, sh.SHAPE_MISMATCH),
    # An unknown format, a rank of 0 or 5, a zero extent, a huge extent.
    ([(1, 0, 7, 1, 0, 4, 1, 1, 1, 0, 16)], 16, sh.UNSUPPORTED_MODEL),
    ([(1, 0, sh.F32, 0, 0, 4, 1, 1, 1, 0, 16)], 16, sh.SHAPE_MISMATCH),
    ([(1, 0, sh.F32, 5, 0, 4, 1, 1, 1, 0, 16)], 16, sh.SHAPE_MISMATCH),
    ([(1, 0, sh.F32, 2, 0, 4, 0, 1, 1, 0, 16)], 16, sh.SHAPE_MISMATCH),
    ([(1, 0, sh.F32, 1, 0, (1 << 24) + 1, 1, 1, 1, 0, 4 * ((1 << 24) + 1))], 16, sh.SHAPE_MISMATCH),
    # Quantized: not a matrix, or a row that is not whole groups.
    ([(1, 0, o.Q4, 1, 0, 64, 1, 1, 1, 0, 34)], 48, sh.SHAPE_MISMATCH),
    ([(1, 0, o.Q4, 2, 0, 1, 96, 1, 1, 0, 64)], 64, sh.SHAPE_MISMATCH),
    # Element tensors of rank 3 and 4 with exact lengths, and bf16 / f16.
    ([(1, 0, sh.F32, 3, 0, 2, 3, 4, 1, 0, 96), (2, 0, sh.BF16, 4, 0, 2, 2, 2, 2, 96, 32),
      (3, 0, sh.F16, 1, 0, 8, 1, 1, 1, 128, 16)], 144, sh.OK),
])
def test_index_rules(entries, payload_len, expected):
    data = entry_shard(entries, payload_len)
    assert statuses(data) == (expected, expected)


def test_multi_tensor_shard_round_trip():
    # Quantized matrices of every format and element vectors over two layers,
    # built by the writer and read back entry by entry.
    rng = np.random.default_rng(3)
    tensors = []
    for layer, (kind, fmt, rows, cols) in enumerate([(sh.KIND_DECODER_Q, o.Q4, 48, 128),
                                                      (sh.KIND_DECODER_K, o.Q5, 16, 192),
                                                      (sh.KIND_DECODER_V, o.Q8, 16, 64)], start=1):
        w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
        scales, data = o.quantize_rows(fmt, w)
        tensors.append(dict(kind=kind, layer=layer, format=fmt, dims=(rows, cols),
                            payload=sh.quantized_payload(fmt, scales, data)))
        norm = rng.standard_normal(cols).astype(np.float32)
        tensors.append(dict(kind=sh.KIND_DECODER_ATTENTION_NORM, layer=layer, format=sh.F32, dims=(cols,),
                            payload=norm.tobytes()))
    data = sh.build(tensors)
    assert qa.shard_validate(data) == (0, len(tensors))
    assert qa.shard_verify_checksum(data) == 0
    payload_offset = struct.unpack_from("<I", data, 16)[0]
    for t in tensors:
        status, entry = qa.shard_find(data, t["kind"], t["layer"])
        assert status == 0 and entry.format == t["format"] and entry.len_bytes == len(t["payload"])
        assert entry.offset_bytes % 16 == 0
        start = payload_offset + entry.offset_bytes
        assert data[start:start + entry.len_bytes] == t["payload"]


def test_tensor_kind_numbering():
    # container.zig:521-549: on-disk values are permanent.
    assert sh.KIND_AUDIO_CONV1_WEIGHT == 1 and sh.KIND_DECODER_EMBED_TOKENS == 30
    assert ((1 << 16) | 30) < ((2 << 16) | 1) and ((0 << 16) | 99) < ((1 << 16) | 1)
