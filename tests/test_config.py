"""config.bin (model_config.zig) on the host: qwh_config_parse and the
oracle's restatement against the reference's own tests (:376-662) and the
decoder dimensions a configuration implies. No device is needed."""
import math

import pytest

import qwenscriber_amd as qa
from oracle import model_config as mc

STATUS = {mc.OK: 0, mc.BAD_MAGIC: -4, mc.BAD_VERSION: -5, mc.TRUNCATED: -11}


def check(config: dict, reason: int):
    data = mc.pack(config)
    assert mc.parse(data) == reason
    status, got, parsed = qa.config_parse(data)
    assert (status, got) == (STATUS.get(reason, -1), reason)
    return parsed


@pytest.mark.parametrize("base", [mc.CONFIG_0P6B, mc.CONFIG_1P7B], ids=["0.6B", "1.7B"])
def test_released_configurations_are_valid(base):
    parsed = check(base, mc.OK)
    dims = qa.config_decoder(parsed)
    assert dims["hidden"] == base["text_hidden_size"] and dims["layers"] == 28 and dims["heads"] == 16
    assert dims["kv_heads"] == 8 and dims["head_dim"] == 128 and dims["ffn"] == base["text_ffn_dim"]
    assert dims["vocab"] == 151936 and dims["max_positions"] == 16384
    assert math.isclose(dims["eps"], 1e-6, rel_tol=1e-6) and dims["theta"] == 1e6
    # model_config.zig:416-437 derived geometry (the decoder's part): query
    # groups 2, query width 2048, key/value width 1024.
    assert dims["heads"] // dims["kv_heads"] == 2
    assert dims["heads"] * dims["head_dim"] == 2048 and dims["kv_heads"] * dims["head_dim"] == 1024


@pytest.mark.parametrize("change,reason", [
    # model_config.zig:525-615, one corruption per check.
    (dict(magic=b"XWCFG001"), mc.BAD_MAGIC),
    (dict(format_version=2), mc.BAD_VERSION),
    (dict(flags=1), mc.OK),                        # tied output projection is a known flag
    (dict(flags=2), mc.RESERVED_NOT_EMPTY),
    (dict(reserved1=1), mc.RESERVED_NOT_EMPTY),
    (dict(architecture=99), mc.UNKNOWN_ARCHITECTURE),
    (dict(audio_attention_heads=13), mc.INVALID_HEAD_GEOMETRY),
    (dict(text_attention_heads=12), mc.INVALID_HEAD_GEOMETRY),
    (dict(text_key_value_heads=5), mc.INVALID_HEAD_GEOMETRY),
    (dict(audio_output_dim=2048), mc.INVALID_DIMENSION),
    (dict(mel_bins=80), mc.INVALID_MEL_GEOMETRY),
    (dict(audio_n_window_infer=850), mc.INVALID_CHUNK_GEOMETRY),
    (dict(audio_max_position_steps=12), mc.INVALID_CHUNK_GEOMETRY),
    (dict(token_audio_pad=151936), mc.INVALID_TOKEN_ID),
    (dict(text_rms_norm_eps=0.0), mc.INVALID_EPSILON),
    (dict(rope_theta=0.5), mc.INVALID_ROPE_THETA),
    (dict(text_layers=0), mc.INVALID_DIMENSION),
    # The remaining checks.
    (dict(text_layers=513), mc.INVALID_DIMENSION),
    (dict(text_head_dim=63), mc.INVALID_HEAD_GEOMETRY),
    (dict(audio_n_window=0), mc.INVALID_CHUNK_GEOMETRY),
    (dict(audio_n_window=1501, audio_n_window_infer=3002), mc.INVALID_CHUNK_GEOMETRY),
    (dict(vocab_size=(1 << 21) + 1), mc.INVALID_DIMENSION),
    (dict(max_positions=0), mc.INVALID_DIMENSION),
    (dict(max_decode_tokens=8193), mc.INVALID_DIMENSION),
    (dict(audio_layer_norm_eps=float("inf")), mc.INVALID_EPSILON),
    (dict(text_rms_norm_eps=float("nan")), mc.INVALID_EPSILON),
    (dict(rope_theta=float("inf")), mc.INVALID_ROPE_THETA),
    (dict(text_ffn_dim=(1 << 24) + 1), mc.INVALID_DIMENSION),
])
def test_invalid_configurations_are_rejected_with_a_reason(change, reason):
    check(dict(mc.CONFIG_0P6B, **change), reason)


def test_parse_enforces_size_and_alignment():
    # model_config.zig:618-662.
    zeros = bytes(160)
    assert mc.parse(zeros) == mc.BAD_MAGIC
    assert qa.config_parse(zeros)[:2] == (-4, mc.BAD_MAGIC)
    good = mc.pack(mc.CONFIG_0P6B)
    assert qa.config_parse(good[:-1])[:2] == (-11, mc.TRUNCATED)
    assert qa.config_parse(good + b"\0")[:2] == (-11, mc.TRUNCATED)
    assert qa.config_parse(good, offset=1)[:2] == (-1, mc.MISALIGNED)
    assert mc.parse(good, aligned=False) == mc.MISALIGNED
    status, reason, parsed = qa.config_parse(good, offset=4)
    assert (status, reason) == (0, mc.OK) and parsed.audio_d_model == 896
