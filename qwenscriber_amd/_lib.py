"""ctypes binding of libqwhip.so (include/qwhip.h).

Names follow the reference's operator surface (kernels.zig Matrix.apply /
linearQuantized / decodeAttentionStepQ8, quant.zig quantizeRow, decoder.zig
forwardToken / step): the methods below are one-line forwards to the C ABI.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

FORMAT_F32, FORMAT_F16 = 0, 1
FORMAT_Q4, FORMAT_Q5, FORMAT_Q8 = 16, 17, 18
GROUP_SIZE = 64
DATA_BYTES = {FORMAT_Q4: 32, FORMAT_Q5: 40, FORMAT_Q8: 64}

T_EMBED, T_Q, T_K, T_V, T_O, T_GATE, T_UP, T_DOWN, T_LM_HEAD = range(9)
T_ATTN_NORM, T_Q_NORM, T_K_NORM, T_FFN_NORM, T_FINAL_NORM = 16, 17, 18, 19, 20
CACHE_F32, CACHE_Q8 = 0, 1

class AudioLayerWeights(ctypes.Structure):
    """qwh_audio_layer_weights (model.zig AudioLayer): matrix handles and
    device addresses of f32 vectors."""

    MATRICES = ("q", "k", "v", "o", "ffn_in", "ffn_out")
    VECTORS = ("q_bias", "k_bias", "v_bias", "o_bias", "ffn_in_bias", "ffn_out_bias", "attention_norm_weight",
               "attention_norm_bias", "final_norm_weight", "final_norm_bias")
    _fields_ = [(name, ctypes.c_uint64) for name in MATRICES] + [(name, ctypes.c_void_p) for name in VECTORS]


class AudioFrontendWeights(ctypes.Structure):
    """qwh_audio_frontend_weights: device addresses of the three f16-bit
    convolution weights and f32 biases, and the conv_out matrix handle."""

    _fields_ = [("conv1_weight", ctypes.c_void_p), ("conv2_weight", ctypes.c_void_p), ("conv3_weight", ctypes.c_void_p),
                ("conv1_bias", ctypes.c_void_p), ("conv2_bias", ctypes.c_void_p), ("conv3_bias", ctypes.c_void_p),
                ("conv_out", ctypes.c_uint64)]


STATUS = {
    0: "ok", -1: "invalid_argument", -2: "out_of_memory", -3: "unsupported", -4: "bad_magic",
    -5: "bad_version", -6: "checksum_mismatch", -7: "shape_mismatch", -8: "invalid_state",
    -9: "limit_exceeded", -10: "not_found", -11: "truncated", -13: "unsupported_model", -64: "device",
}


def library_path() -> str:
    return os.environ.get("QWHIP_LIBRARY", os.path.join(HERE, "build", "libqwhip.so"))


class QwhError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS.get(status, status)} ({status}): {message}")
        self.status = status


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


class TensorEntry(ctypes.Structure):
    """qwh_tensor_entry: one `.qw` index entry (container.zig Entry)."""
    _fields_ = [
        ("kind", ctypes.c_uint16),
        ("layer", ctypes.c_uint16),
        ("format", ctypes.c_uint8),
        ("rank", ctypes.c_uint8),
        ("reserved", ctypes.c_uint16),
        ("dims", ctypes.c_uint32 * 4),
        ("offset_bytes", ctypes.c_uint64),
        ("len_bytes", ctypes.c_uint64),
    ]


class ModelConfig(ctypes.Structure):
    """qwh_model_config: config.bin's 160-byte model_config.Config."""
    _fields_ = [("magic", ctypes.c_char * 8), ("format_version", ctypes.c_uint32), ("architecture", ctypes.c_uint32)] + [
        (name, ctypes.c_uint32) for name in (
            "audio_d_model", "audio_layers", "audio_attention_heads", "audio_ffn_dim",
            "audio_downsample_hidden_size", "audio_n_window", "audio_n_window_infer",
            "audio_max_position_steps", "audio_output_dim", "mel_bins")
    ] + [("audio_layer_norm_eps", ctypes.c_float)] + [
        (name, ctypes.c_uint32) for name in (
            "text_hidden_size", "text_layers", "text_attention_heads", "text_key_value_heads",
            "text_head_dim", "text_ffn_dim", "vocab_size")
    ] + [("text_rms_norm_eps", ctypes.c_float), ("rope_theta", ctypes.c_float)] + [
        (name, ctypes.c_uint32) for name in (
            "max_positions", "max_decode_tokens", "token_audio_start", "token_audio_end", "token_audio_pad",
            "token_im_start", "token_im_end", "token_endoftext", "token_asr_text", "token_eos_primary",
            "token_eos_secondary", "token_pad", "flags")
    ] + [("reserved", ctypes.c_uint32 * 3)]


_P = ctypes.c_void_p
_PP = ctypes.POINTER(ctypes.c_void_p)
_U16 = ctypes.c_uint16
_U32 = ctypes.c_uint32
_U64 = ctypes.c_uint64
_I32 = ctypes.c_int32
_F = ctypes.c_float

# Every entry point of include/qwhip.h with its ctypes signature.
SIGNATURES = {
    "qwh_abi_version": (_I32, []),
    "qwh_status_string": (ctypes.c_char_p, [_I32]),
    "qwh_create": (_I32, [_U32, _PP]),
    "qwh_destroy": (_I32, [_P]),
    "qwh_sync": (_I32, [_P]),
    "qwh_last_error": (ctypes.c_char_p, [_P]),
    "qwh_device_cus": (_I32, [_P, ctypes.POINTER(_U32)]),
    "qwh_alloc": (_I32, [_P, _U64, _PP]),
    "qwh_free": (_I32, [_P, _P]),
    "qwh_upload": (_I32, [_P, _P, _P, _U64]),
    "qwh_download": (_I32, [_P, _P, _P, _U64]),
    "qwh_memset": (_I32, [_P, _P, _I32, _U64]),
    "qwh_event_record": (_I32, [_P, _U32]),
    "qwh_stream_read": (_I32, [_P, _P, _U64, _U32, _P]),
    "qwh_conv3x3s2_gelu": (_I32, [_P, _P, _P, _P, _P, _U32, _U32, _U32, _U32, _U32]),
    "qwh_audio_frontend": (_I32, [_P, ctypes.POINTER(AudioFrontendWeights), _P, _U32, _U32, _U32, _U32, _U32, _P, _U32,
                                  ctypes.POINTER(_U32)]),
    "qwh_event_elapsed": (_I32, [_P, _U32, _U32, ctypes.POINTER(_F)]),
    "qwh_matrix_upload": (_I32, [_P, _I32, _U32, _U32, _P, _U64, _P, _U64, ctypes.POINTER(_U64)]),
    "qwh_matrix_wrap": (_I32, [_P, _I32, _U32, _U32, _P, _P, ctypes.POINTER(_U64)]),
    "qwh_matrix_synthetic": (_I32, [_P, _I32, _U32, _U32, _U32, _U32, _F, ctypes.POINTER(_U64)]),
    "qwh_matrix_planes": (_I32, [_P, _U64, _PP, _PP]),
    "qwh_matrix_release": (_I32, [_P, _U64]),
    "qwh_linear": (_I32, [_P, _U64, _P, _U32, _U32, _P]),
    "qwh_linear_bf16": (_I32, [_P, _U64, _P, _U32, _U32, _P]),
    "qwh_activation_bytes": (_I32, [_U32, _U32, ctypes.POINTER(_U64)]),
    "qwh_activation_prepare": (_I32, [_P, _P, _U32, _U32, _P]),
    "qwh_linear_prepared": (_I32, [_P, _U64, _P, _U32, _P]),
    "qwh_quantize_rows": (_I32, [_P, _I32, _P, _U32, _U32, _P, _P]),
    "qwh_synth_normal": (_I32, [_P, _U32, _U32, _U64, _F, _P]),
    "qwh_decode_attention_q8": (_I32, [_P, _P, _P, _P, _P, _P, _P, _U32, _U32, _U32, _U32, _U32, _U64, _U64]),
    "qwh_kv_append_q8": (_I32, [_P, _P, _P, _U32, _U32, _P, _P, _P, _P]),
    "qwh_argmax_rows": (_I32, [_P, _P, _U32, _U32, _P]),
    "qwh_layer_norm": (_I32, [_P, _P, _P, _P, _P, _U32, _U32, _F]),
    "qwh_add_bias": (_I32, [_P, _P, _P, _U32, _U32]),
    "qwh_gelu": (_I32, [_P, _P, _U64]),
    "qwh_audio_attention_window": (_I32, [_P, _P, _U32, _P, _U32, _P, _U32, _P, _U32, _U32, _U32, _U32, _U32]),
    "qwh_audio_attention": (_I32, [_P, _P, _U32, _P, _P, _P, _U32, _U32, _U32, _U32, _U32]),
    "qwh_audio_layer": (_I32, [_P, ctypes.POINTER(AudioLayerWeights), _P, _U32, _U32, _U32, _U32, _U32, _F]),
    "qwh_audio_projector": (_I32, [_P, _U64, _P, _U64, _P, _P, _U32, _P]),
    "qwh_decoder_create": (_I32, [_P, ctypes.POINTER(DecoderConfig), _U32, _PP]),
    "qwh_decoder_create_cache": (_I32, [_P, ctypes.POINTER(DecoderConfig), _U32, _U32, _PP]),
    "qwh_decoder_init_synthetic_format": (_I32, [_P, _U32, _I32]),
    "qwh_decoder_generate_until": (_I32, [_P, _P, _U32, _P, _U32, _P, _P]),
    "qwh_decode_attention_f32": (_I32, [_P, _P, _P, _P, _P, _U32, _U32, _U32, _U32, _U32, _U64]),
    "qwh_decode_attention_q8_noalloc": (_I32, [_P, _P, _P, _P, _P, _P, _P, _U32, _U32, _U32, _U32, _U32, _U64, _U64]),
    "qwh_decoder_destroy": (_I32, [_P]),
    "qwh_decoder_set_matrix": (_I32, [_P, _U32, _U32, _U64]),
    "qwh_decoder_set_vector": (_I32, [_P, _U32, _U32, _P, _U32]),
    "qwh_decoder_init_synthetic": (_I32, [_P, _U32]),
    "qwh_decoder_reset": (_I32, [_P]),
    "qwh_decoder_prefill_random": (_I32, [_P, _U32, _U32, _U32]),
    "qwh_decoder_cache_planes": (_I32, [_P, _U32, _U32, _PP, _PP, _PP, _PP]),
    "qwh_decoder_position": (_I32, [_P, _U32, ctypes.POINTER(_U32)]),
    "qwh_decoder_set_position": (_I32, [_P, _U32, _U32]),
    "qwh_decoder_forward": (_I32, [_P, _P, _I32]),
    "qwh_decoder_forward_rows": (_I32, [_P, _P, _P, _P, _I32]),
    "qwh_decoder_prefill": (_I32, [_P, _U32, _P, _U32, _U32, _P, _U32, _P]),
    "qwh_decoder_step": (_I32, [_P, _P, _P]),
    "qwh_decoder_generate": (_I32, [_P, _P, _U32, _P]),
    "qwh_decoder_logits": (_I32, [_P, _U32, _P, _U32]),
    "qwh_shard_validate": (_I32, [_P, _U64, ctypes.POINTER(_U32)]),
    "qwh_shard_verify_checksum": (_I32, [_P, _U64]),
    "qwh_shard_find": (_I32, [_P, _U64, _U16, _U16, ctypes.POINTER(TensorEntry)]),
    "qwh_shard_load": (_I32, [_P, _P, _U64, ctypes.POINTER(_U64)]),
    "qwh_shard_tensor": (_I32, [_P, _U64, _U16, _U16, _PP, ctypes.POINTER(TensorEntry)]),
    "qwh_shard_matrix": (_I32, [_P, _U64, _U16, _U16, ctypes.POINTER(_U64)]),
    "qwh_shard_release": (_I32, [_P, _U64]),
    "qwh_decoder_bind_shard": (_I32, [_P, _U64, _U32, ctypes.POINTER(_U32)]),
    "qwh_config_parse": (_I32, [_P, _U64, ctypes.POINTER(ModelConfig), ctypes.POINTER(_U32)]),
    "qwh_config_decoder": (_I32, [ctypes.POINTER(ModelConfig), ctypes.POINTER(DecoderConfig)]),
}

_lib = None


def load():
    """Loads libqwhip.so; raises if it is not built (no fallback exists)."""
    global _lib
    if _lib is None:
        path = library_path()
        if not os.path.exists(path):
            raise RuntimeError(
                f"libqwhip.so not found at {path}: build it with `make -C qwenscriber_amd` "
                "(or __graft_entry__.build()). There is no CPU fallback.")
        lib = ctypes.CDLL(path)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
    return _lib


def _bytes_arg(data) -> tuple:
    buf = np.frombuffer(bytes(data), np.uint8) if not isinstance(data, np.ndarray) else np.ascontiguousarray(data, np.uint8)
    return buf, buf.ctypes.data, buf.size


def config_parse(data, offset: int = 0) -> tuple:
    """qwh_config_parse: (status, reason, ModelConfig or None). `offset`
    shifts the bytes inside a 16-byte aligned buffer (alignment checks)."""
    raw = bytes(data)
    buf = np.zeros(len(raw) + 16, np.uint8)
    base = (-buf.ctypes.data) % 16 + offset
    if base + len(raw) > buf.size:
        base -= 16
    buf[base:base + len(raw)] = np.frombuffer(raw, np.uint8)
    out = ModelConfig()
    reason = ctypes.c_uint32(0)
    status = load().qwh_config_parse(buf.ctypes.data + base, len(raw), ctypes.byref(out), ctypes.byref(reason))
    return status, reason.value, (out if status == 0 else None)


def config_decoder(model: "ModelConfig") -> dict:
    """Decoder(**config) keyword arguments of a parsed configuration."""
    out = DecoderConfig()
    status = load().qwh_config_decoder(ctypes.byref(model), ctypes.byref(out))
    if status != 0:
        raise QwhError(status, "qwh_config_decoder")
    return {name: getattr(out, name) for name, _ in DecoderConfig._fields_}


def shard_validate(data) -> tuple:
    """qwh_shard_validate on host bytes: (status, tensor_count). No device."""
    buf, ptr, n = _bytes_arg(data)
    count = ctypes.c_uint32(0)
    status = load().qwh_shard_validate(ptr, n, ctypes.byref(count))
    return status, count.value


def shard_verify_checksum(data) -> int:
    buf, ptr, n = _bytes_arg(data)
    return load().qwh_shard_verify_checksum(ptr, n)


def shard_find(data, kind: int, layer: int) -> tuple:
    """qwh_shard_find: (status, TensorEntry or None)."""
    buf, ptr, n = _bytes_arg(data)
    entry = TensorEntry()
    status = load().qwh_shard_find(ptr, n, kind, layer, ctypes.byref(entry))
    return status, (entry if status == 0 else None)


def _ptr(array: np.ndarray) -> int:
    if not array.flags["C_CONTIGUOUS"]:
        raise ValueError("array must be C contiguous")
    return array.ctypes.data


class DeviceBuffer:
    """A device allocation owned by a Context (qwh_alloc / qwh_free)."""

    def __init__(self, ctx: "Context", nbytes: int):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        out = ctypes.c_void_p()
        ctx._check(load().qwh_alloc(ctx.handle, self.nbytes, ctypes.byref(out)))
        self.ptr = out.value

    def free(self) -> None:
        if self.ptr is not None and self.ctx.handle:
            self.ctx._check(load().qwh_free(self.ctx.handle, self.ptr))
        self.ptr = None

    def upload(self, array: np.ndarray, offset: int = 0) -> None:
        array = np.ascontiguousarray(array)
        if offset + array.nbytes > self.nbytes:
            raise ValueError("upload past the end of the buffer")
        self.ctx._check(load().qwh_upload(self.ctx.handle, self.ptr + offset, _ptr(array), array.nbytes))

    def download(self, dtype, count: Optional[int] = None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype)
        if offset + out.nbytes > self.nbytes:
            raise ValueError("download past the end of the buffer")
        self.ctx._check(load().qwh_download(self.ctx.handle, _ptr(out), self.ptr + offset, out.nbytes))
        return out


class Context:
    """One device and one stream (qwh_create)."""

    def __init__(self, device: int = 0):
        self.lib = load()
        out = ctypes.c_void_p()
        status = self.lib.qwh_create(device, ctypes.byref(out))
        if status != 0:
            raise QwhError(status, f"qwh_create({device}) failed")
        self.handle = out.value
        self._buffers = []

    def close(self) -> None:
        if self.handle:
            self.lib.qwh_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _check(self, status: int) -> None:
        if status != 0:
            message = self.lib.qwh_last_error(self.handle).decode() if self.handle else ""
            raise QwhError(status, message)

    # -- memory and timing -------------------------------------------------
    def buffer(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def memset(self, dev: int, value: int, nbytes: int) -> None:
        self._check(self.lib.qwh_memset(self.handle, dev, value, nbytes))

    def to_device(self, array: np.ndarray) -> DeviceBuffer:
        array = np.ascontiguousarray(array)
        buf = DeviceBuffer(self, max(array.nbytes, 1))
        buf.upload(array)
        return buf

    def sync(self) -> None:
        self._check(self.lib.qwh_sync(self.handle))

    def cus(self) -> int:
        out = ctypes.c_uint32()
        self._check(self.lib.qwh_device_cus(self.handle, ctypes.byref(out)))
        return out.value

    def event_record(self, slot: int) -> None:
        self._check(self.lib.qwh_event_record(self.handle, slot))

    def stream_read(self, src_dev: int, nbytes: int, blocks_per_cu: int, sink_dev: int) -> None:
        self._check(self.lib.qwh_stream_read(self.handle, src_dev, nbytes, blocks_per_cu, sink_dev))

    def event_elapsed_ms(self, start: int, end: int) -> float:
        out = ctypes.c_float()
        self._check(self.lib.qwh_event_elapsed(self.handle, start, end, ctypes.byref(out)))
        return out.value

    # -- matrices (kernels.zig Matrix) ------------------------------------
    def matrix_upload(self, fmt: int, rows: int, cols: int, scales: Optional[np.ndarray], data: np.ndarray) -> int:
        """Quantized planes, or for f32 / f16 (scales None) the elements as
        bytes or as a float32 / uint16 array."""
        data = np.ascontiguousarray(data).reshape(-1).view(np.uint8)
        out = ctypes.c_uint64()
        if scales is None:
            s_ptr, s_len = None, 0
        else:
            scales = np.ascontiguousarray(scales, np.uint8)
            s_ptr, s_len = _ptr(scales), scales.size
        self._check(self.lib.qwh_matrix_upload(self.handle, fmt, rows, cols, s_ptr, s_len,
                                               _ptr(data), data.size, ctypes.byref(out)))
        return out.value

    def matrix_wrap(self, fmt: int, rows: int, cols: int, scales_dev: int, data_dev: int) -> int:
        out = ctypes.c_uint64()
        self._check(self.lib.qwh_matrix_wrap(self.handle, fmt, rows, cols, scales_dev, data_dev, ctypes.byref(out)))
        return out.value

    def matrix_synthetic(self, fmt: int, rows: int, cols: int, seed: int, stream: int, scale: float = 0.02) -> int:
        out = ctypes.c_uint64()
        self._check(self.lib.qwh_matrix_synthetic(self.handle, fmt, rows, cols, seed, stream, scale, ctypes.byref(out)))
        return out.value

    # -- `.qw` shards (container.zig) -------------------------------------
    def shard_load(self, data) -> int:
        buf, ptr, n = _bytes_arg(data)
        out = ctypes.c_uint64()
        self._check(self.lib.qwh_shard_load(self.handle, ptr, n, ctypes.byref(out)))
        return out.value

    def shard_tensor(self, shard: int, kind: int, layer: int):
        dev = ctypes.c_void_p()
        entry = TensorEntry()
        self._check(self.lib.qwh_shard_tensor(self.handle, shard, kind, layer, ctypes.byref(dev), ctypes.byref(entry)))
        return dev.value, entry

    def shard_matrix(self, shard: int, kind: int, layer: int) -> int:
        out = ctypes.c_uint64()
        self._check(self.lib.qwh_shard_matrix(self.handle, shard, kind, layer, ctypes.byref(out)))
        return out.value

    def shard_release(self, shard: int) -> None:
        self._check(self.lib.qwh_shard_release(self.handle, shard))

    def matrix_planes(self, matrix: int):
        s = ctypes.c_void_p()
        d = ctypes.c_void_p()
        self._check(self.lib.qwh_matrix_planes(self.handle, matrix, ctypes.byref(s), ctypes.byref(d)))
        return s.value, d.value

    def matrix_release(self, matrix: int) -> None:
        self._check(self.lib.qwh_matrix_release(self.handle, matrix))

    def linear(self, matrix: int, x_dev: int, cols: int, tokens: int, out_dev: int) -> None:
        """kernels.zig Matrix.apply: out[tokens][rows] = W x."""
        self._check(self.lib.qwh_linear(self.handle, matrix, x_dev, cols, tokens, out_dev))

    def activation_bytes(self, cols: int, tokens: int) -> int:
        out = ctypes.c_uint64()
        self._check(self.lib.qwh_activation_bytes(cols, tokens, ctypes.byref(out)))
        return out.value

    def activation_prepare(self, x_dev: int, cols: int, tokens: int, prepared_dev: int) -> None:
        self._check(self.lib.qwh_activation_prepare(self.handle, x_dev, cols, tokens, prepared_dev))

    def linear_prepared(self, matrix: int, prepared_dev: int, tokens: int, out_dev: int) -> None:
        self._check(self.lib.qwh_linear_prepared(self.handle, matrix, prepared_dev, tokens, out_dev))

    def linear_bf16(self, matrix: int, x_dev: int, cols: int, tokens: int, out_dev: int) -> None:
        self._check(self.lib.qwh_linear_bf16(self.handle, matrix, x_dev, cols, tokens, out_dev))

    # -- audio tower (model.zig:646-735) -----------------------------------
    def layer_norm(self, out_dev: int, x_dev: int, weight_dev: int, bias_dev: int, width: int, tokens: int,
                   eps: float) -> None:
        """kernels.zig layerNormInto (out may equal x: layerNorm in place)."""
        self._check(self.lib.qwh_layer_norm(self.handle, out_dev, x_dev, weight_dev, bias_dev, width, tokens, eps))

    def add_bias(self, x_dev: int, bias_dev: int, rows: int, tokens: int) -> None:
        """kernels.zig addBias."""
        self._check(self.lib.qwh_add_bias(self.handle, x_dev, bias_dev, rows, tokens))

    def gelu(self, x_dev: int, count: int) -> None:
        """math.zig gelu over count values in place."""
        self._check(self.lib.qwh_gelu(self.handle, x_dev, count))

    def audio_attention_window(self, out_dev, out_stride, q_dev, q_stride, k_dev, k_stride, v_dev, v_stride,
                               window_start, window_length, heads, head_dim) -> None:
        """kernels.zig audioAttentionWindow."""
        self._check(self.lib.qwh_audio_attention_window(self.handle, out_dev, out_stride, q_dev, q_stride, k_dev,
                                                        k_stride, v_dev, v_stride, window_start, window_length,
                                                        heads, head_dim))

    def audio_attention(self, out_dev, out_stride, q_dev, k_dev, v_dev, qkv_stride, steps, window_steps, heads,
                        head_dim) -> None:
        """model.zig runWindowedAttention: every window in one launch."""
        self._check(self.lib.qwh_audio_attention(self.handle, out_dev, out_stride, q_dev, k_dev, v_dev, qkv_stride,
                                                 steps, window_steps, heads, head_dim))

    def audio_layer(self, weights: "AudioLayerWeights", encoder_dev: int, steps: int, d_model: int, heads: int,
                    ffn_dim: int, window_steps: int, eps: float) -> None:
        """model.zig runAudioTower, one layer over encoder[steps][d_model] in place."""
        self._check(self.lib.qwh_audio_layer(self.handle, ctypes.byref(weights), encoder_dev, steps, d_model, heads,
                                             ffn_dim, window_steps, eps))

    def audio_projector(self, in_matrix, in_bias_dev, out_matrix, out_bias_dev, encoder_dev, steps, out_dev) -> None:
        """model.zig runProjector."""
        self._check(self.lib.qwh_audio_projector(self.handle, in_matrix, in_bias_dev, out_matrix, out_bias_dev,
                                                 encoder_dev, steps, out_dev))

    def conv3x3s2_gelu(self, out_dev, in_dev, weights_dev, bias_dev, batch, out_channels, in_channels, in_height,
                       in_width) -> None:
        """kernels.zig conv3x3Stride2Gelu over `batch` images."""
        self._check(self.lib.qwh_conv3x3s2_gelu(self.handle, out_dev, in_dev, weights_dev, bias_dev, batch, out_channels,
                                                in_channels, in_height, in_width))

    def audio_frontend(self, weights, log_mel_dev, mel_bins, frames, n_window, downsample, d_model, encoder_dev,
                       encoder_rows) -> int:
        """model.zig convolveAndPack: returns the number of encoder rows written."""
        steps = ctypes.c_uint32(0)
        self._check(self.lib.qwh_audio_frontend(self.handle, ctypes.byref(weights), log_mel_dev, mel_bins, frames,
                                                n_window, downsample, d_model, encoder_dev, encoder_rows,
                                                ctypes.byref(steps)))
        return steps.value

    # -- quantization and synthetic inputs ---------------------------------
    def quantize_rows(self, fmt: int, values_dev: int, rows: int, cols: int, scales_dev: int, data_dev: int) -> None:
        self._check(self.lib.qwh_quantize_rows(self.handle, fmt, values_dev, rows, cols, scales_dev, data_dev))

    def synth_normal(self, seed: int, stream: int, count: int, scale: float, out_dev: int) -> None:
        self._check(self.lib.qwh_synth_normal(self.handle, seed, stream, count, scale, out_dev))

    # -- attention ----------------------------------------------------------
    def decode_attention_f32(self, out_dev, query_dev, keys_dev, values_dev, cached, heads, kv_heads, head_dim,
                             batch=1, stride=0):
        self._check(self.lib.qwh_decode_attention_f32(self.handle, out_dev, query_dev, keys_dev, values_dev, cached,
                                                      heads, kv_heads, head_dim, batch, stride))

    def decode_attention_q8(self, out_dev, query_dev, k_scales, k_codes, v_scales, v_codes, cached, heads,
                            kv_heads, head_dim, batch=1, scale_stride=0, code_stride=0) -> None:
        self._check(self.lib.qwh_decode_attention_q8(self.handle, out_dev, query_dev, k_scales, k_codes, v_scales,
                                                     v_codes, cached, heads, kv_heads, head_dim, batch,
                                                     scale_stride, code_stride))

    def kv_append_q8(self, key_dev, value_dev, kv_width, position, k_scales, k_codes, v_scales, v_codes) -> None:
        self._check(self.lib.qwh_kv_append_q8(self.handle, key_dev, value_dev, kv_width, position, k_scales,
                                              k_codes, v_scales, v_codes))

    def argmax_rows(self, logits_dev: int, rows: int, count: int, ids_dev: int) -> None:
        """decoder.zig:290-301 argmaxLogits of each of `rows` rows (qwh_argmax_rows)."""
        self._check(self.lib.qwh_argmax_rows(self.handle, logits_dev, rows, count, ids_dev))


class Decoder:
    """decoder.zig Decoder over `batch` sequences (qwh_decoder_*), with a q8
    (CACHE_Q8, the default here) or f32 (CACHE_F32) key/value cache."""

    def __init__(self, ctx: Context, batch: int = 1, cache_format: int = CACHE_Q8, **config):
        self.ctx = ctx
        self.config = DecoderConfig(**config)
        self.batch = batch
        self.cache_format = cache_format
        out = ctypes.c_void_p()
        ctx._check(ctx.lib.qwh_decoder_create_cache(ctx.handle, ctypes.byref(self.config), batch, cache_format,
                                                    ctypes.byref(out)))
        self.handle = out.value

    def close(self) -> None:
        if self.handle:
            self.ctx.lib.qwh_decoder_destroy(self.handle)
            self.handle = None

    def _check(self, status):
        self.ctx._check(status)

    def set_matrix(self, kind: int, layer: int, matrix: int) -> None:
        self._check(self.ctx.lib.qwh_decoder_set_matrix(self.handle, kind, layer, matrix))

    def set_vector(self, kind: int, layer: int, values: np.ndarray) -> None:
        values = np.ascontiguousarray(values, np.float32)
        self._check(self.ctx.lib.qwh_decoder_set_vector(self.handle, kind, layer, _ptr(values), values.size))

    def bind_shard(self, shard: int, output_tied: bool = False) -> int:
        bound = ctypes.c_uint32(0)
        self._check(self.ctx.lib.qwh_decoder_bind_shard(self.handle, shard, 1 if output_tied else 0, ctypes.byref(bound)))
        return bound.value

    def init_synthetic(self, seed: int, fmt: int = FORMAT_Q4) -> None:
        self._check(self.ctx.lib.qwh_decoder_init_synthetic_format(self.handle, seed, fmt))

    def reset(self) -> None:
        self._check(self.ctx.lib.qwh_decoder_reset(self.handle))

    def prefill_random(self, seq: int, count: int, seed: int) -> None:
        self._check(self.ctx.lib.qwh_decoder_prefill_random(self.handle, seq, count, seed))

    def cache_planes(self, seq: int, layer: int):
        ptrs = [ctypes.c_void_p() for _ in range(4)]
        self._check(self.ctx.lib.qwh_decoder_cache_planes(self.handle, seq, layer, *[ctypes.byref(p) for p in ptrs]))
        return tuple(p.value for p in ptrs)

    def position(self, seq: int) -> int:
        out = ctypes.c_uint32()
        self._check(self.ctx.lib.qwh_decoder_position(self.handle, seq, ctypes.byref(out)))
        return out.value

    def set_position(self, seq: int, position: int) -> None:
        self._check(self.ctx.lib.qwh_decoder_set_position(self.handle, seq, position))

    def forward(self, tokens, want_logits: bool = True) -> None:
        tokens = np.ascontiguousarray(tokens, np.uint32)
        self._check(self.ctx.lib.qwh_decoder_forward(self.handle, _ptr(tokens), int(want_logits)))

    def forward_rows(self, tokens, rows_dev: int, mask=None, want_logits: bool = True) -> None:
        """forwardToken with audio rows (batch x hidden f32 on the device) in
        place of the embeddings of the sequences `mask` selects (all if None)."""
        tokens = np.ascontiguousarray(tokens, np.uint32)
        m = None if mask is None else np.ascontiguousarray(np.asarray(mask, bool).astype(np.uint8))
        self._check(self.ctx.lib.qwh_decoder_forward_rows(self.handle, _ptr(tokens), rows_dev,
                                                          None if m is None else _ptr(m), int(want_logits)))

    def prefill(self, seq: int, tokens, audio_pad: int = 0xFFFFFFFF, audio_rows_dev: int = 0,
                audio_steps: int = 0) -> int:
        """Decoder.prefill (decoder.zig:308-333) of one sequence: the prompt
        tokens, audio pads taking the device audio rows in order; returns the
        greedy next token."""
        tokens = np.ascontiguousarray(tokens, np.uint32)
        out = np.zeros(1, np.uint32)
        self._check(self.ctx.lib.qwh_decoder_prefill(self.handle, seq, _ptr(tokens), tokens.size, audio_pad,
                                                     audio_rows_dev or None, audio_steps, _ptr(out)))
        return int(out[0])

    def step(self, tokens) -> np.ndarray:
        tokens = np.ascontiguousarray(tokens, np.uint32)
        out = np.zeros(self.batch, np.uint32)
        self._check(self.ctx.lib.qwh_decoder_step(self.handle, _ptr(tokens), _ptr(out)))
        return out

    def generate(self, tokens, steps: int) -> np.ndarray:
        tokens = np.ascontiguousarray(tokens, np.uint32)
        out = np.zeros(steps * self.batch, np.uint32)
        self._check(self.ctx.lib.qwh_decoder_generate(self.handle, _ptr(tokens), steps, _ptr(out)))
        return out.reshape(steps, self.batch)

    def generate_until(self, tokens, max_tokens: int, stop_tokens=()):
        """qwh_decoder_generate_until: (ids [max_tokens x batch], counts [batch])."""
        tokens = np.ascontiguousarray(tokens, np.uint32)
        stops = np.ascontiguousarray(list(stop_tokens) or [0], np.uint32)
        ids = np.zeros(max(1, max_tokens) * self.batch, np.uint32)
        counts = np.zeros(self.batch, np.uint32)
        self._check(self.ctx.lib.qwh_decoder_generate_until(self.handle, _ptr(tokens), max_tokens, _ptr(stops),
                                                            len(stop_tokens), _ptr(ids), _ptr(counts)))
        return ids[: max_tokens * self.batch].reshape(max_tokens, self.batch), counts

    def logits(self, seq: int) -> np.ndarray:
        out = np.zeros(self.config.vocab, np.float32)
        self._check(self.ctx.lib.qwh_decoder_logits(self.handle, seq, _ptr(out), out.size))
        return out
