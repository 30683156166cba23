"""config.bin restated in plain Python. TEST INFRASTRUCTURE.

Only tests/ may import this module, as the checker of the library's
qwh_config_parse and as the writer of the configurations it reads. It follows
src/core/model_config.zig: the 160-byte Config layout (:110-190, offsets
asserted at :362-374), parse (:354-360) and Config.validate (:260-327), with
the reasons in model_config.Error's order (:89-106).
"""
from __future__ import annotations

import math
import struct

(OK, BAD_MAGIC, BAD_VERSION, TRUNCATED, RESERVED_NOT_EMPTY, UNKNOWN_ARCHITECTURE, INVALID_DIMENSION,
 INVALID_HEAD_GEOMETRY, INVALID_MEL_GEOMETRY, INVALID_TOKEN_ID, INVALID_EPSILON, INVALID_ROPE_THETA,
 INVALID_CHUNK_GEOMETRY, MISALIGNED) = range(14)

FIELDS = [  # (name, struct code) in on-disk order after magic
    ("format_version", "I"), ("architecture", "I"),
    ("audio_d_model", "I"), ("audio_layers", "I"), ("audio_attention_heads", "I"), ("audio_ffn_dim", "I"),
    ("audio_downsample_hidden_size", "I"), ("audio_n_window", "I"), ("audio_n_window_infer", "I"),
    ("audio_max_position_steps", "I"), ("audio_output_dim", "I"), ("mel_bins", "I"), ("audio_layer_norm_eps", "f"),
    ("text_hidden_size", "I"), ("text_layers", "I"), ("text_attention_heads", "I"), ("text_key_value_heads", "I"),
    ("text_head_dim", "I"), ("text_ffn_dim", "I"), ("vocab_size", "I"), ("text_rms_norm_eps", "f"),
    ("rope_theta", "f"), ("max_positions", "I"), ("max_decode_tokens", "I"),
    ("token_audio_start", "I"), ("token_audio_end", "I"), ("token_audio_pad", "I"), ("token_im_start", "I"),
    ("token_im_end", "I"), ("token_endoftext", "I"), ("token_asr_text", "I"), ("token_eos_primary", "I"),
    ("token_eos_secondary", "I"), ("token_pad", "I"), ("flags", "I"),
    ("reserved1", "I"), ("reserved2", "I"), ("reserved3", "I"),
]
LAYOUT = "<8s" + "".join(code for _, code in FIELDS)

# The released checkpoints' configurations (model_config.zig:376-470).
TOKENS = dict(token_audio_start=151669, token_audio_end=151670, token_audio_pad=151676, token_im_start=151644,
              token_im_end=151645, token_endoftext=151643, token_asr_text=151704, token_eos_primary=151643,
              token_eos_secondary=151645, token_pad=151643)
CONFIG_0P6B = dict(magic=b"QWCFG001", format_version=1, architecture=1, audio_d_model=896, audio_layers=18,
                   audio_attention_heads=14, audio_ffn_dim=3584, audio_downsample_hidden_size=480, audio_n_window=50,
                   audio_n_window_infer=800, audio_max_position_steps=13, audio_output_dim=1024, mel_bins=128,
                   audio_layer_norm_eps=1e-5, text_hidden_size=1024, text_layers=28, text_attention_heads=16,
                   text_key_value_heads=8, text_head_dim=128, text_ffn_dim=3072, vocab_size=151936,
                   text_rms_norm_eps=1e-6, rope_theta=1e6, max_positions=16384, max_decode_tokens=256,
                   flags=0, reserved1=0, reserved2=0, reserved3=0, **TOKENS)
CONFIG_1P7B = dict(CONFIG_0P6B, audio_d_model=1024, audio_layers=24, audio_attention_heads=16, audio_ffn_dim=4096,
                   audio_output_dim=2048, text_hidden_size=2048, text_ffn_dim=6144)


def pack(config: dict) -> bytes:
    return struct.pack(LAYOUT, config["magic"], *[config[name] for name, _ in FIELDS])


def unpack(data: bytes) -> dict:
    values = struct.unpack(LAYOUT, data)
    return dict(magic=values[0], **{name: v for (name, _), v in zip(FIELDS, values[1:])})


def _steps(n: int) -> int:
    for _ in range(3):
        n = (n - 1) // 2 + 1
    return n


def validate(c: dict) -> int:
    if c["magic"] != b"QWCFG001":
        return BAD_MAGIC
    if c["format_version"] != 1:
        return BAD_VERSION
    if c["flags"] & ~1 or c["reserved1"] or c["reserved2"] or c["reserved3"]:
        return RESERVED_NOT_EMPTY
    if c["architecture"] != 1:
        return UNKNOWN_ARCHITECTURE
    ranged = ("audio_d_model", "audio_ffn_dim", "audio_downsample_hidden_size", "audio_output_dim",
              "text_hidden_size", "text_ffn_dim", "text_head_dim")
    if any(not 0 < c[k] <= 1 << 24 for k in ranged):
        return INVALID_DIMENSION
    if any(not 0 < c[k] <= 512 for k in ("audio_layers", "text_layers")):
        return INVALID_DIMENSION
    if c["mel_bins"] != 128:
        return INVALID_MEL_GEOMETRY
    heads = c["audio_attention_heads"]
    if heads == 0 or c["audio_d_model"] % heads:
        return INVALID_HEAD_GEOMETRY
    if c["audio_d_model"] // heads < 2 or (c["audio_d_model"] // heads) % 2:
        return INVALID_HEAD_GEOMETRY
    th, kv = c["text_attention_heads"], c["text_key_value_heads"]
    if th == 0 or kv == 0 or th % kv:
        return INVALID_HEAD_GEOMETRY
    if c["text_head_dim"] < 2 or c["text_head_dim"] % 2:
        return INVALID_HEAD_GEOMETRY
    if c["text_hidden_size"] != c["audio_output_dim"]:
        return INVALID_DIMENSION
    if c["audio_n_window"] == 0:
        return INVALID_CHUNK_GEOMETRY
    chunk = 2 * c["audio_n_window"]
    if chunk > 480000 // 160 or c["audio_n_window_infer"] % chunk or c["audio_max_position_steps"] < _steps(chunk):
        return INVALID_CHUNK_GEOMETRY
    if c["mel_bins"] % 8:
        return INVALID_MEL_GEOMETRY
    if not 0 < c["vocab_size"] <= 1 << 21 or not 0 < c["max_positions"] <= 1 << 24:
        return INVALID_DIMENSION
    if not 0 < c["max_decode_tokens"] <= 8192:
        return INVALID_DIMENSION
    ae, te = c["audio_layer_norm_eps"], c["text_rms_norm_eps"]
    if not math.isfinite(ae) or not math.isfinite(te) or not ae > 0 or not te > 0:
        return INVALID_EPSILON
    if not math.isfinite(c["rope_theta"]) or not c["rope_theta"] > 1.0:
        return INVALID_ROPE_THETA
    if any(c[k] >= c["vocab_size"] for k in TOKENS):
        return INVALID_TOKEN_ID
    return OK


def parse(data: bytes, aligned: bool = True) -> int:
    if len(data) != 160:
        return TRUNCATED
    if not aligned:
        return MISALIGNED
    return validate(unpack(data))
