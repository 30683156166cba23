"""`.qw` shard reader and writer in plain Python. TEST INFRASTRUCTURE.

Only tests/ may import this module, as the checker of the library's shard
entry points and as the writer of the shards they read. It restates
src/core/container.zig (File.parse / validate / find / checksum, :175-290,
Header.validate :88-99, Entry.validate :142-160) and the one-tensor builder of
its tests (:553-582) for several tensors, with the statuses wasm/abi.zig:90-146
gives File.parse's errors.
"""
from __future__ import annotations

import struct

from . import oracle as o

OK, INVALID_ARGUMENT, BAD_MAGIC, BAD_VERSION, CHECKSUM_MISMATCH = 0, -1, -4, -5, -6
SHAPE_MISMATCH, NOT_FOUND, TRUNCATED, UNSUPPORTED_MODEL = -7, -10, -11, -13

MAGIC = b"QWSHARD1"
HEADER_BYTES = 32
ENTRY_BYTES = 40
PAYLOAD_ALIGN = 256
TENSOR_ALIGN = 16
F32, F16, BF16 = 0, 1, 2
ELEMENT_BYTES = {F32: 4, F16: 2, BF16: 2}
QUANTIZED = (o.Q4, o.Q5, o.Q8)

# container.TensorKind values used by the tests (container.zig:337-381).
KIND_AUDIO_CONV1_WEIGHT = 1
KIND_AUDIO_CONV2_WEIGHT = 3
KIND_DECODER_EMBED_TOKENS = 30
KIND_DECODER_FINAL_NORM = 31
KIND_DECODER_OUTPUT = 32
KIND_DECODER_Q = 33
KIND_DECODER_K = 34
KIND_DECODER_V = 35
KIND_DECODER_ATTENTION_NORM = 39
KIND_DECODER_FFN_DOWN = 43


def _up(value: int, alignment: int) -> int:
    return -(-value // alignment) * alignment


def quantized_len(fmt: int, rows: int, cols: int, base: int = 0):
    """quant.planeLayout(fmt, rows, cols, base, 16): (scales offset, data
    offset, total), offsets relative to base."""
    groups = rows * cols // 64
    scales_off = _up(base, TENSOR_ALIGN) - base
    data_off = _up(base + scales_off + 2 * groups, TENSOR_ALIGN) - base
    return scales_off, data_off, data_off + groups * o.DATA_BYTES[fmt]


def _entry_status(kind, layer, fmt, rank, dims, offset, length) -> int:
    if fmt not in ELEMENT_BYTES and fmt not in QUANTIZED:
        return UNSUPPORTED_MODEL
    if not 1 <= rank <= 4 or any(d == 0 or d > (1 << 24) for d in dims[:rank]):
        return SHAPE_MISMATCH
    if fmt in QUANTIZED:
        if rank != 2 or dims[1] % 64:
            return SHAPE_MISMATCH
        if quantized_len(fmt, dims[0], dims[1])[2] != length:
            return SHAPE_MISMATCH
        scales_off, _, total = quantized_len(fmt, dims[0], dims[1], offset)
        if total != length or scales_off != 0:
            return SHAPE_MISMATCH
        return OK
    count = 1
    for d in dims[:rank]:
        count *= d
    if count * ELEMENT_BYTES[fmt] >= 1 << 64 or count * ELEMENT_BYTES[fmt] != length:
        return SHAPE_MISMATCH
    return OK


def parse(data: bytes):
    """(status, entries): entries as (kind, layer, fmt, rank, dims, offset,
    length) tuples when the shard is valid."""
    if len(data) < HEADER_BYTES:
        return TRUNCATED, None
    if data[:8] != MAGIC:
        return BAD_MAGIC, None
    version, index_len, payload_offset, payload_len, count, _ = struct.unpack_from("<6I", data, 8)
    if version != 1:
        return BAD_VERSION, None
    if index_len != count * ENTRY_BYTES or payload_offset < HEADER_BYTES + index_len or payload_offset % PAYLOAD_ALIGN:
        return TRUNCATED, None
    if len(data) < HEADER_BYTES + index_len or len(data) < payload_offset + payload_len:
        return TRUNCATED, None
    entries = []
    previous_end = 0
    previous_key = None
    for i in range(count):
        kind, layer, fmt, rank, _reserved = struct.unpack_from("<HHBBH", data, HEADER_BYTES + i * ENTRY_BYTES)
        dims = struct.unpack_from("<4I", data, HEADER_BYTES + i * ENTRY_BYTES + 8)
        offset, length = struct.unpack_from("<2Q", data, HEADER_BYTES + i * ENTRY_BYTES + 24)
        status = _entry_status(kind, layer, fmt, rank, dims, offset, length)
        if status != OK:
            return status, None
        key = (layer << 16) | kind
        if previous_key is not None and key <= previous_key:
            return INVALID_ARGUMENT, None
        previous_key = key
        if offset < previous_end:
            return INVALID_ARGUMENT, None
        if offset + length > payload_len:
            return TRUNCATED, None
        previous_end = offset + length
        if offset % TENSOR_ALIGN:
            return INVALID_ARGUMENT, None
        entries.append((kind, layer, fmt, rank, dims, offset, length))
    return OK, entries


def find(entries, kind: int, layer: int):
    for entry in entries:
        if (entry[1], entry[0]) == (layer, kind):
            return entry
    return None


def checksum(payload: bytes) -> int:
    """Low 32 bits of FNV-1a 64 (container.zig:279-281)."""
    return o.fnv1a64(payload) & 0xFFFFFFFF


def verify_checksum(data: bytes) -> int:
    status, _ = parse(data)
    if status != OK:
        return status
    payload_offset, payload_len = struct.unpack_from("<2I", data, 16)
    recorded = struct.unpack_from("<I", data, 28)[0]
    return OK if checksum(data[payload_offset:payload_offset + payload_len]) == recorded else CHECKSUM_MISMATCH


def build(tensors) -> bytes:
    """A shard of `tensors`: dicts with kind, layer, format, dims and payload
    (bytes: for a quantized matrix, scales then data at planeLayout's
    offsets). Entries sorted by (layer, kind), each payload at the next
    16-byte boundary, the payload section at a 256-byte boundary."""
    tensors = sorted(tensors, key=lambda t: (t["layer"], t["kind"]))
    index = b""
    payload = b""
    for t in tensors:
        offset = _up(len(payload), TENSOR_ALIGN)
        payload += b"\0" * (offset - len(payload)) + bytes(t["payload"])
        dims = list(t["dims"]) + [1] * (4 - len(t["dims"]))
        index += struct.pack("<HHBBH4I2Q", t["kind"], t["layer"], t["format"], len(t["dims"]), 0, *dims,
                             offset, len(t["payload"]))
    payload_offset = _up(HEADER_BYTES + len(index), PAYLOAD_ALIGN)
    header = MAGIC + struct.pack("<6I", 1, len(index), payload_offset, len(payload), len(tensors), checksum(payload))
    return header + index + b"\0" * (payload_offset - HEADER_BYTES - len(index)) + payload


def quantized_payload(fmt: int, scales, data) -> bytes:
    """One quantized matrix's payload: its scale plane, zero padding to the
    next 16-byte boundary, its data plane."""
    scales = bytes(scales)
    return scales + b"\0" * (_up(len(scales), TENSOR_ALIGN) - len(scales)) + bytes(data)
