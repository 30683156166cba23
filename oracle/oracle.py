"""ctypes binding of the CPU oracle (oracle/build/libqwref.so). TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the checker or the timed CPU baseline. The functions
mirror the reference's Zig kernels; see qwref.c for the file:line each follows.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "libqwref.so")

F32, F16 = 0, 1
Q4, Q5, Q8 = 16, 17, 18
GROUP = 64
# Cache formats (model_config.zig:44-68 CacheFormat).
CACHE_F32, CACHE_Q8 = 0, 1
# Norm vector kinds (the library's QWH_T_* values for the same tensors).
ATTN_NORM, Q_NORM, K_NORM, FFN_NORM, FINAL_NORM = 16, 17, 18, 19, 20
DATA_BYTES = {Q4: 32, Q5: 40, Q8: 64}


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


class Layout(ctypes.Structure):
    _fields_ = [
        ("scales_offset_bytes", ctypes.c_uint64),
        ("scales_len_bytes", ctypes.c_uint64),
        ("data_offset_bytes", ctypes.c_uint64),
        ("data_len_bytes", ctypes.c_uint64),
        ("total_len_bytes", ctypes.c_uint64),
        ("group_count", ctypes.c_uint32),
        ("groups_per_row", ctypes.c_uint32),
    ]


class DecoderConfig(ctypes.Structure):
    _fields_ = [
        ("hidden", ctypes.c_uint32),
        ("layers", ctypes.c_uint32),
        ("heads", ctypes.c_uint32),
        ("kv_heads", ctypes.c_uint32),
        ("head_dim", ctypes.c_uint32),
        ("ffn", ctypes.c_uint32),
        ("vocab", ctypes.c_uint32),
        ("max_positions", ctypes.c_uint32),
        ("eps", ctypes.c_float),
        ("theta", ctypes.c_float),
    ]


_P = ctypes.c_void_p
_U8 = ctypes.c_uint8
_U16 = ctypes.c_uint16
_U32 = ctypes.c_uint32
_U64 = ctypes.c_uint64
_I32 = ctypes.c_int32
_F = ctypes.c_float

_SIGNATURES = {
    "qwref_to_f16": (_U16, [_F]),
    "qwref_from_f16": (_F, [_U16]),
    "qwref_to_bf16": (_U16, [_F]),
    "qwref_from_bf16": (_F, [_U16]),
    "qwref_bias": (_I32, [_I32]),
    "qwref_data_bytes_per_group": (_I32, [_I32]),
    "qwref_plane_layout": (_I32, [_I32, _U32, _U32, _U64, _U64, ctypes.POINTER(Layout)]),
    "qwref_plane_bytes": (_U64, [_I32, _U32, _U32]),
    "qwref_quantize_row": (None, [_I32, _P, _U32, _P, _P]),
    "qwref_quantize_rows": (None, [_I32, _P, _U32, _U32, _P, _P]),
    "qwref_dequantize_row": (None, [_I32, _P, _P, _P, _U32]),
    "qwref_dot_row": (_F, [_I32, _P, _P, _P, _U32]),
    "qwref_quant_hash": (_U64, []),
    "qwref_fnv1a64": (_U64, [_P, _U64, _U64]),
    "qwref_dot_f32": (_F, [_P, _P, _U32]),
    "qwref_linear_quantized": (_I32, [_P, _P, _I32, _P, _U64, _P, _U64, _U32, _U32, _U32]),
    "qwref_linear_f32": (_I32, [_P, _P, _P, _U32, _U32, _U32]),
    "qwref_linear_f16": (_I32, [_P, _P, _P, _U32, _U32, _U32]),
    "qwref_embedding_row": (_I32, [_I32, _P, _P, _U32, _U32, _U32, _P]),
    "qwref_add_in_place": (None, [_P, _P, _U32]),
    "qwref_silu_mul": (None, [_P, _P, _P, _U32]),
    "qwref_silu": (_F, [_F]),
    "qwref_softmax_in_place": (None, [_P, _U32]),
    "qwref_rms_norm": (None, [_P, _P, _U32, _U32, _F]),
    "qwref_inverse_frequency": (_F, [_U32, _U32, _F]),
    "qwref_build_rope_tables": (None, [_P, _P, _U32, _F, _U32, _U32]),
    "qwref_rope_in_place": (None, [_P, _P, _U32, _U32, _U32, _P, _P, _U32]),
    "qwref_decode_attention_step": (_I32, [_P, _P, _P, _P, _U32, _U32, _U32, _U32]),
    "qwref_decode_attention_step_q8": (_I32, [_P, _P, _P, _P, _P, _P, _U32, _U32, _U32, _U32]),
    "qwref_argmax": (_U32, [_P, _U32]),
    "qwref_mulberry32_at": (_U32, [_U32, _U64]),
    "qwref_normal_at": (_F, [_U32, _U32, _U64]),
    "qwref_fill_normal": (None, [_P, _U64, _U32, _U32, _F]),
    "qwref_stream_base": (_U32, [_U32, _U32]),
    "qwref_decoder_create_synthetic": (_P, [ctypes.POINTER(DecoderConfig), _U32, _U32]),
    "qwref_decoder_destroy": (None, [_P]),
    "qwref_decoder_create_synthetic_as": (_P, [_P, _U32, _U32, _I32, _I32]),
    "qwref_decoder_set_vector": (_I32, [_P, _U32, _U32, _P, _U32]),
    "qwref_decoder_prefill_random": (_I32, [_P, _U32, _U32]),
    "qwref_decoder_forward": (_I32, [_P, _U32, _U32, _I32]),
    "qwref_decoder_forward_row": (_I32, [_P, _U32, _U32, _P, _I32]),
    "qwref_decoder_logits": (ctypes.POINTER(ctypes.c_float), [_P, _U32]),
    "qwref_decoder_position": (_U32, [_P, _U32]),
    "qwref_decoder_step": (_I32, [_P, _U32, _U32, ctypes.POINTER(_U32)]),
    "qwref_decoder_weights_hash": (_U64, [_P]),
    "qwref_decoder_cache_hash": (_U64, [_P, _U32]),
    "qwref_decoder_cache_row": (_U64, [_P, _U32, _U32, _U32, _P, _U64]),
    "qwref_decoder_set_cache_row": (_I32, [_P, _U32, _U32, _U32, _P, _U64]),
    "qwref_decoder_set_position": (_I32, [_P, _U32, _U32]),
    "qwref_synthetic_start_token": (_U32, [_U32, _U32, _U32]),
    "qwref_set_threads": (None, [_I32]),
    "qwref_erf": (ctypes.c_float, [ctypes.c_float]),
    "qwref_gelu": (ctypes.c_float, [ctypes.c_float]),
    "qwref_gelu_in_place": (None, [_P, _U64]),
    "qwref_add_bias": (_I32, [_P, _P, _U32, _U32]),
    "qwref_layer_norm": (None, [_P, _P, _P, _U32, _U32, ctypes.c_float]),
    "qwref_audio_attention_window": (_I32, [_P, _U32, _P, _U32, _P, _U32, _P, _U32, _U32, _U32, _U32, _U32]),
    "qwref_post_convolution_steps": (_U32, [_U32]),
    "qwref_conv3x3s2_gelu": (_I32, [_P, _P, _P, _P, _U32, _U32, _U32, _U32]),
    "qwref_add_sinusoidal_position": (None, [_P, _U32, _U32]),
}


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        handle = ctypes.CDLL(LIB_PATH)
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def _ptr(array: np.ndarray) -> int:
    assert array.flags["C_CONTIGUOUS"]
    return array.ctypes.data


def set_threads(n: int) -> None:
    lib().qwref_set_threads(int(n))


def to_f16(value: float) -> int:
    return lib().qwref_to_f16(value)


def from_f16(bits: int) -> float:
    return lib().qwref_from_f16(bits)


def quant_hash() -> int:
    return lib().qwref_quant_hash()


def fnv1a64(data: bytes | np.ndarray, state: int = 0xCBF29CE484222325) -> int:
    buf = np.ascontiguousarray(np.frombuffer(bytes(data), np.uint8) if isinstance(data, bytes) else data).view(np.uint8)
    return lib().qwref_fnv1a64(_ptr(buf), buf.size, state)


def plane_layout(fmt: int, rows: int, cols: int, base: int = 0, alignment: int = 16):
    out = Layout()
    status = lib().qwref_plane_layout(fmt, rows, cols, base, alignment, ctypes.byref(out))
    return status, out


def plane_bytes(fmt: int, positions: int, cols: int) -> int:
    return lib().qwref_plane_bytes(fmt, positions, cols)


def quantize_rows(fmt: int, values: np.ndarray):
    """quantizeRow per row: returns (scales u8 [rows*gpr*2], data u8)."""
    values = np.ascontiguousarray(values, dtype=np.float32)
    rows, cols = values.shape if values.ndim == 2 else (1, values.shape[0])
    gpr = cols // GROUP
    scales = np.zeros(rows * gpr * 2, np.uint8)
    data = np.zeros(rows * gpr * DATA_BYTES[fmt], np.uint8)
    lib().qwref_quantize_rows(fmt, _ptr(values), rows, cols, _ptr(scales), _ptr(data))
    return scales, data


def dequantize_rows(fmt: int, scales: np.ndarray, data: np.ndarray, rows: int, cols: int) -> np.ndarray:
    gpr = cols // GROUP
    out = np.zeros((rows, cols), np.float32)
    for r in range(rows):
        s = np.ascontiguousarray(scales[r * gpr * 2:(r + 1) * gpr * 2])
        d = np.ascontiguousarray(data[r * gpr * DATA_BYTES[fmt]:(r + 1) * gpr * DATA_BYTES[fmt]])
        row = np.zeros(cols, np.float32)
        lib().qwref_dequantize_row(fmt, _ptr(s), _ptr(d), _ptr(row), cols)
        out[r] = row
    return out


def dot_row(fmt: int, scales: np.ndarray, data: np.ndarray, x: np.ndarray) -> float:
    x = np.ascontiguousarray(x, np.float32)
    return lib().qwref_dot_row(fmt, _ptr(np.ascontiguousarray(scales)), _ptr(np.ascontiguousarray(data)), _ptr(x), x.size)


def dot_f32(a: np.ndarray, b: np.ndarray) -> float:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return lib().qwref_dot_f32(_ptr(a), _ptr(b), a.size)


def linear_quantized(fmt: int, scales: np.ndarray, data: np.ndarray, rows: int, cols: int,
                     x: np.ndarray, tokens: int = 1) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.zeros(tokens * rows, np.float32)
    scales = np.ascontiguousarray(scales)
    data = np.ascontiguousarray(data)
    status = lib().qwref_linear_quantized(_ptr(out), _ptr(x), fmt, _ptr(scales), scales.size,
                                          _ptr(data), data.size, rows, cols, tokens)
    if status != 0:
        raise ValueError(f"linear_quantized status {status}")
    return out.reshape(tokens, rows)


def linear_f32(weights: np.ndarray, x: np.ndarray, tokens: int = 1) -> np.ndarray:
    weights = np.ascontiguousarray(weights, np.float32)
    rows, cols = weights.shape
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.zeros(tokens * rows, np.float32)
    lib().qwref_linear_f32(_ptr(out), _ptr(x), _ptr(weights), rows, cols, tokens)
    return out.reshape(tokens, rows)


def linear_f16(weights: np.ndarray, x: np.ndarray, tokens: int = 1) -> np.ndarray:
    """kernels.zig:82-112 linearF16 over f16 bit patterns [rows, cols] (uint16)."""
    weights = np.ascontiguousarray(weights, np.uint16)
    rows, cols = weights.shape
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.zeros(tokens * rows, np.float32)
    status = lib().qwref_linear_f16(_ptr(out), _ptr(x), _ptr(weights), rows, cols, tokens)
    if status != 0:
        raise ValueError(f"linear_f16 status {status}")
    return out.reshape(tokens, rows)


def embedding_row(fmt: int, scales, data, rows: int, cols: int, row: int) -> np.ndarray:
    """decoder.zig:346-376 embeddingRow: row `row` of a matrix in `fmt` (f32
    values or f16 bits as `data` for the element formats, scales None)."""
    out = np.zeros(cols, np.float32)
    data = np.ascontiguousarray(data).reshape(-1).view(np.uint8)
    s_ptr = None if scales is None else _ptr(np.ascontiguousarray(scales, np.uint8))
    status = lib().qwref_embedding_row(fmt, s_ptr, _ptr(data), rows, cols, row, _ptr(out))
    if status != 0:
        raise ValueError(f"embedding_row status {status}")
    return out


def linear_any(fmt: int, scales, data, rows: int, cols: int, x: np.ndarray, tokens: int = 1) -> np.ndarray:
    """kernels.zig:182-206 Matrix.apply: the arm of the matrix's storage.
    Quantized (fmt, scales, data) planes, or f32 values / f16 bits as `data`
    (scales None) for the element formats."""
    if fmt == F32:
        return linear_f32(np.asarray(data, np.float32).reshape(rows, cols), x, tokens)
    if fmt == F16:
        return linear_f16(np.asarray(data).reshape(-1).view(np.uint16).reshape(rows, cols), x, tokens)
    return linear_quantized(fmt, scales, data, rows, cols, x, tokens)


def silu(x: float) -> float:
    return lib().qwref_silu(x)


def silu_mul(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    gate = np.ascontiguousarray(gate, np.float32)
    up = np.ascontiguousarray(up, np.float32)
    out = np.zeros_like(gate)
    lib().qwref_silu_mul(_ptr(out), _ptr(gate), _ptr(up), gate.size)
    return out


def softmax(row: np.ndarray) -> np.ndarray:
    row = np.array(row, np.float32)
    lib().qwref_softmax_in_place(_ptr(row), row.size)
    return row


def rms_norm(x: np.ndarray, weight: np.ndarray, width: int, eps: float) -> np.ndarray:
    x = np.array(x, np.float32).reshape(-1)
    weight = np.ascontiguousarray(weight, np.float32)
    lib().qwref_rms_norm(_ptr(x), _ptr(weight), width, x.size // width, eps)
    return x


def inverse_frequency(index: int, head_dim: int, theta: float) -> float:
    return lib().qwref_inverse_frequency(index, head_dim, theta)


def rope_tables(half: int, theta: float, max_positions: int):
    cos = np.zeros(max_positions * half, np.float32)
    sin = np.zeros(max_positions * half, np.float32)
    lib().qwref_build_rope_tables(_ptr(cos), _ptr(sin), half, theta, max_positions, half)
    return cos, sin


def rope(x: np.ndarray, positions, heads: int, head_dim: int, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    x = np.array(x, np.float32).reshape(-1)
    positions = np.ascontiguousarray(positions, np.uint32)
    lib().qwref_rope_in_place(_ptr(x), _ptr(positions), positions.size, heads, head_dim, _ptr(cos), _ptr(sin), head_dim // 2)
    return x


def decode_attention(query, keys, values, cached, heads, kv_heads, head_dim) -> np.ndarray:
    query = np.ascontiguousarray(query, np.float32)
    keys = np.ascontiguousarray(keys, np.float32)
    values = np.ascontiguousarray(values, np.float32)
    out = np.zeros(heads * head_dim, np.float32)
    status = lib().qwref_decode_attention_step(_ptr(out), _ptr(query), _ptr(keys), _ptr(values), cached, heads, kv_heads, head_dim)
    if status != 0:
        raise ValueError(f"decode_attention status {status}")
    return out


def decode_attention_q8(query, k_scales, k_codes, v_scales, v_codes, cached, heads, kv_heads, head_dim) -> np.ndarray:
    arrays = [np.ascontiguousarray(a) for a in (query, k_scales, k_codes, v_scales, v_codes)]
    out = np.zeros(heads * head_dim, np.float32)
    status = lib().qwref_decode_attention_step_q8(_ptr(out), *[_ptr(a) for a in arrays], cached, heads, kv_heads, head_dim)
    if status != 0:
        raise ValueError(f"decode_attention_q8 status {status}")
    return out


def argmax(logits: np.ndarray) -> int:
    logits = np.ascontiguousarray(logits, np.float32)
    return lib().qwref_argmax(_ptr(logits), logits.size)


def mulberry32_at(base: int, draw: int) -> int:
    return lib().qwref_mulberry32_at(base, draw)


def stream_base(seed: int, stream: int) -> int:
    return lib().qwref_stream_base(seed, stream)


def normal(count: int, seed: int, stream: int = 0, scale: float = 1.0) -> np.ndarray:
    out = np.zeros(count, np.float32)
    lib().qwref_fill_normal(_ptr(out), count, seed, stream, scale)
    return out


class Decoder:
    """decoder.zig restatement over a synthetic model: every linear in
    `weight_format` (q4 by default), the cache in `cache_format` (q8 by
    default), norm weights 1.0 until set_vector replaces them."""

    def __init__(self, seed: int, batch: int = 1, weight_format: int = Q4, cache_format: int = CACHE_Q8,
                 **config):
        self.config = DecoderConfig(**config)
        self.handle = lib().qwref_decoder_create_synthetic_as(ctypes.byref(self.config), seed, batch,
                                                              weight_format, cache_format)
        if not self.handle:
            raise ValueError(f"unsupported formats {weight_format} / {cache_format}")
        self.seed = seed
        self.batch = batch
        self.weight_format = weight_format
        self.cache_format = cache_format

    def set_vector(self, kind: int, layer: int, values) -> None:
        values = np.ascontiguousarray(values, np.float32)
        status = lib().qwref_decoder_set_vector(self.handle, kind, layer, _ptr(values), values.size)
        if status != 0:
            raise ValueError(f"set_vector status {status}")

    def close(self):
        if self.handle:
            lib().qwref_decoder_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()

    def prefill_random(self, seq: int, count: int) -> None:
        assert lib().qwref_decoder_prefill_random(self.handle, seq, count) == 0

    def forward(self, seq: int, token: int, want_logits: bool = True) -> None:
        status = lib().qwref_decoder_forward(self.handle, seq, token, int(want_logits))
        if status != 0:
            raise ValueError(f"forward status {status}")

    def forward_row(self, seq: int, token: int, row: np.ndarray, want_logits: bool = True) -> None:
        """forwardToken with an audio row in place of the token's embedding."""
        row = np.ascontiguousarray(row, np.float32)
        status = lib().qwref_decoder_forward_row(self.handle, seq, token, _ptr(row), int(want_logits))
        if status != 0:
            raise ValueError(f"forward_row status {status}")

    def logits(self, seq: int) -> np.ndarray:
        ptr = lib().qwref_decoder_logits(self.handle, seq)
        return np.ctypeslib.as_array(ptr, shape=(self.config.vocab,)).copy()

    def position(self, seq: int) -> int:
        return lib().qwref_decoder_position(self.handle, seq)

    def step(self, seq: int, token: int) -> int:
        out = ctypes.c_uint32(0)
        status = lib().qwref_decoder_step(self.handle, seq, token, ctypes.byref(out))
        if status != 0:
            raise ValueError(f"step status {status}")
        return out.value

    def weights_hash(self) -> int:
        return lib().qwref_decoder_weights_hash(self.handle)

    def cache_hash(self, seq: int) -> int:
        return lib().qwref_decoder_cache_hash(self.handle, seq)

    def cache_row(self, seq: int, layer: int, position: int) -> bytes:
        """One cache row as the decoder holds it: q8 key scales, key codes,
        value scales, value codes (f32 cache: key row, value row)."""
        kvw = self.config.kv_heads * self.config.head_dim
        out = np.zeros(8 * kvw, np.uint8)
        n = lib().qwref_decoder_cache_row(self.handle, seq, layer, position, out.ctypes.data, out.size)
        if n == 0:
            raise ValueError("cache_row: bad argument")
        return out[:n].tobytes()

    def set_cache_row(self, seq: int, layer: int, position: int, row) -> None:
        """Stores a row in cache_row's layout (test plumbing: the next
        forward reads exactly these bytes)."""
        buf = np.ascontiguousarray(np.frombuffer(bytes(row), np.uint8))
        status = lib().qwref_decoder_set_cache_row(self.handle, seq, layer, position, buf.ctypes.data, buf.size)
        if status != 0:
            raise ValueError(f"set_cache_row status {status}")

    def set_position(self, seq: int, position: int) -> None:
        status = lib().qwref_decoder_set_position(self.handle, seq, position)
        if status != 0:
            raise ValueError(f"set_position status {status}")


def start_token(seed: int, seq: int, vocab: int) -> int:
    return lib().qwref_synthetic_start_token(seed, seq, vocab)


# --------------------------------------------------------------------------
# Audio tower (model.zig:646-735): the layer and projector are composed here
# from the C restatements above, call for call in the reference's order.


def erf(x: float) -> float:
    return lib().qwref_erf(float(x))


def gelu(x: float) -> float:
    return lib().qwref_gelu(float(x))


def gelu_array(x: np.ndarray) -> np.ndarray:
    out = np.array(x, np.float32)
    lib().qwref_gelu_in_place(_ptr(out), out.size)
    return out


def add_bias(x: np.ndarray, bias: np.ndarray, rows: int, tokens: int) -> np.ndarray:
    """kernels.zig:210-218 addBias, on a copy."""
    out = np.array(x, np.float32).reshape(-1)
    bias = np.ascontiguousarray(bias, np.float32)
    if out.size != rows * tokens or bias.size != rows:
        raise ValueError("add_bias shape mismatch")
    lib().qwref_add_bias(_ptr(out), _ptr(bias), rows, tokens)
    return out


def layer_norm(x: np.ndarray, weight: np.ndarray, bias: np.ndarray, width: int, eps: float) -> np.ndarray:
    """kernels.zig:259-271 layerNormInto (math.zig:99-116 per row), on a copy."""
    out = np.array(x, np.float32).reshape(-1)
    weight = np.ascontiguousarray(weight, np.float32)
    bias = np.ascontiguousarray(bias, np.float32)
    lib().qwref_layer_norm(_ptr(out), _ptr(weight), _ptr(bias), width, out.size // width, float(eps))
    return out


def audio_attention_window(out, q, k, v, strides, window_start, window_length, heads, head_dim) -> None:
    """kernels.zig:429-484 audioAttentionWindow into `out` (f32, modified in place)."""
    arrays = [np.ascontiguousarray(a, np.float32) for a in (q, k, v)]
    assert out.dtype == np.float32 and out.flags["C_CONTIGUOUS"]
    so, sq, sk, sv = strides
    status = lib().qwref_audio_attention_window(_ptr(out), so, _ptr(arrays[0]), sq, _ptr(arrays[1]), sk,
                                                _ptr(arrays[2]), sv, window_start, window_length, heads, head_dim)
    if status != 0:
        raise ValueError(f"audio_attention_window status {status}")


def audio_attention(q, k, v, steps, window_steps, heads, head_dim) -> np.ndarray:
    """model.zig:792-822 runWindowedAttention over separate [steps][heads*head_dim]
    q, k, v rows: windows of window_steps from step 0, the last one ragged."""
    width = heads * head_dim
    out = np.zeros(steps * width, np.float32)
    start = 0
    while start < steps:
        length = min(window_steps, steps - start)
        audio_attention_window(out, q, k, v, (width, width, width, width), start, length, heads, head_dim)
        start += length
    return out


def audio_layer(encoder: np.ndarray, layer: dict, steps: int, d_model: int, heads: int, ffn_dim: int,
                window_steps: int, eps: float) -> np.ndarray:
    """One audio tower layer (model.zig:656-693 runAudioTower loop body).

    `layer` holds (fmt, scales, data) triples (linear_any) under q, k, v, o, ffn_in, ffn_out
    and f32 vectors under q_bias ... ffn_out_bias, attention_norm_weight / _bias
    and final_norm_weight / _bias. Returns the new residual stream."""
    enc = np.array(encoder, np.float32).reshape(-1)

    def apply(name, x, rows, cols):
        fmt, scales, data = layer[name]
        return linear_any(fmt, scales, data, rows, cols, x, steps).reshape(-1)

    normed = layer_norm(enc, layer["attention_norm_weight"], layer["attention_norm_bias"], d_model, eps)
    # model.zig:765-786 projectQkv: each projection, then its bias.
    q = add_bias(apply("q", normed, d_model, d_model), layer["q_bias"], d_model, steps)
    k = add_bias(apply("k", normed, d_model, d_model), layer["k_bias"], d_model, steps)
    v = add_bias(apply("v", normed, d_model, d_model), layer["v_bias"], d_model, steps)
    block = audio_attention(q, k, v, steps, window_steps, heads, d_model // heads)
    # model.zig:824-848 projectAttentionOutput, then :669 addInPlace.
    block = add_bias(apply("o", block, d_model, d_model), layer["o_bias"], d_model, steps)
    lib().qwref_add_in_place(_ptr(enc), _ptr(block), enc.size)
    normed = layer_norm(enc, layer["final_norm_weight"], layer["final_norm_bias"], d_model, eps)
    # model.zig:852-872 activateFfn, then :692 addInPlace.
    wide = gelu_array(add_bias(apply("ffn_in", normed, ffn_dim, d_model), layer["ffn_in_bias"], ffn_dim, steps))
    block = add_bias(apply("ffn_out", wide, d_model, ffn_dim), layer["ffn_out_bias"], d_model, steps)
    lib().qwref_add_in_place(_ptr(enc), _ptr(block), enc.size)
    return enc


def audio_projector(encoder: np.ndarray, proj_in, in_bias, proj_out, out_bias, steps: int, d_model: int,
                    hidden: int) -> np.ndarray:
    """model.zig:707-735 runProjector: linear, bias, GELU, linear, bias.
    proj_in / proj_out are (fmt, scales, data) (linear_any); proj_in is [d_model x d_model]."""
    fmt, scales, data = proj_in
    mid = linear_any(fmt, scales, data, d_model, d_model, np.asarray(encoder, np.float32), steps)
    mid = gelu_array(add_bias(mid, in_bias, d_model, steps))
    fmt, scales, data = proj_out
    out = linear_any(fmt, scales, data, hidden, d_model, mid, steps)
    return add_bias(out, out_bias, hidden, steps)


# --------------------------------------------------------------------------
# Audio convolution front end (model.zig:509-644 convolveAndPack and
# projectConvStep), composed from the C restatements in the reference's order.


def post_convolution_steps(frames: int) -> int:
    return lib().qwref_post_convolution_steps(frames)


def conv3x3s2_gelu(x: np.ndarray, weights_f16: np.ndarray, bias: np.ndarray, out_channels: int, in_channels: int,
                   in_height: int, in_width: int) -> np.ndarray:
    """kernels.zig:325-427 over one image: x [in][h][w] f32, weights
    [out][in][3][3] f16 bits; returns [out][oh][ow]."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    w = np.ascontiguousarray(weights_f16, np.uint16).reshape(-1)
    b = np.ascontiguousarray(bias, np.float32)
    oh, ow = (in_height - 1) // 2 + 1, (in_width - 1) // 2 + 1
    out = np.zeros(out_channels * oh * ow, np.float32)
    status = lib().qwref_conv3x3s2_gelu(_ptr(out), _ptr(x), _ptr(w), _ptr(b), out_channels, in_channels, in_height,
                                        in_width)
    if status != 0:
        raise ValueError(f"conv status {status}")
    return out.reshape(out_channels, oh, ow)


def add_sinusoidal_position(row: np.ndarray, step: int) -> np.ndarray:
    row = np.array(row, np.float32).reshape(-1)
    lib().qwref_add_sinusoidal_position(_ptr(row), step, row.size)
    return row


def audio_frontend(log_mel: np.ndarray, mel_bins: int, frames: int, n_window: int, weights: dict,
                   downsample: int, d_model: int) -> np.ndarray:
    """model.zig:509-644: per chunk of 2 * n_window frames (the tail zero
    filled), three conv3x3Stride2Gelu stages, then per valid time step the
    (channel, frequency) flatten, the conv_out projection
    (weights["conv_out"] = (format, scales, data)) and the sinusoidal
    position of the step within its chunk. log_mel is [mel_bins][frames]."""
    log_mel = np.asarray(log_mel, np.float32).reshape(mel_bins, frames)
    chunk_frames = 2 * n_window
    chunk_steps = post_convolution_steps(chunk_frames)
    bins = post_convolution_steps(mel_bins)
    features = downsample * bins
    fmt, scales, data = weights["conv_out"]
    rows = []
    for start in range(0, frames, chunk_frames):
        valid = min(frames - start, chunk_frames)
        chunk = np.zeros((mel_bins, chunk_frames), np.float32)
        chunk[:, :valid] = log_mel[:, start:start + valid]
        h, w = mel_bins, chunk_frames
        x = chunk
        for stage, channels in (("conv1", 1), ("conv2", downsample), ("conv3", downsample)):
            x = conv3x3s2_gelu(x, weights[stage + "_weight"], weights[stage + "_bias"], downsample, channels, h, w)
            h, w = (h - 1) // 2 + 1, (w - 1) // 2 + 1
        for step in range(min(chunk_steps, post_convolution_steps(valid))):
            flat = np.ascontiguousarray(x[:, :, step].reshape(features))
            row = linear_any(fmt, scales, data, d_model, features, flat, 1)[0]
            rows.append(add_sinusoidal_position(row, step))
    return np.stack(rows) if rows else np.zeros((0, d_model), np.float32)
