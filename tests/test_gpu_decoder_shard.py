"""A decoder bound from `.qw` shards (qwh_decoder_bind_shard, container.zig
TensorKind 30..43) runs the same model as one bound tensor by tensor: the
synthetic model's exact planes (q4) or elements (f16, the converter's
--quantization none) and norm weights written into two shards give
bit-identical logits and the same greedy token ids."""
import numpy as np
import pytest

import qwenscriber_amd as qa
from oracle import model_config as mc
from oracle import shard as sh

pytestmark = pytest.mark.gpu

TINY = dict(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=128, ffn=512, vocab=1000,
            max_positions=64, eps=1e-6, theta=1e6)
SEED = 13
# Decoder slots (include/qwhip.h QWH_T_*).
T_EMBED, T_Q, T_K, T_V, T_O, T_GATE, T_UP, T_DOWN, T_LM_HEAD = range(9)
T_ATTN_NORM, T_Q_NORM, T_K_NORM, T_FFN_NORM, T_FINAL_NORM = 16, 17, 18, 19, 20


def planes(ctx, rows, cols, stream, fmt):
    """The synthetic generator's matrix in `fmt` (the streams init_synthetic
    uses) as a shard payload."""
    m = ctx.matrix_synthetic(fmt, rows, cols, SEED, stream, 0.02)
    sp, dp = ctx.matrix_planes(m)
    if fmt == qa.FORMAT_F16:
        bits = np.empty(rows * cols, np.uint16)
        ctx._check(ctx.lib.qwh_download(ctx.handle, bits.ctypes.data, dp, bits.nbytes))
        ctx.matrix_release(m)
        return bits.tobytes()
    groups = rows * cols // 64
    s = np.empty(groups * 2, np.uint8)
    d = np.empty(groups * 32, np.uint8)
    ctx._check(ctx.lib.qwh_download(ctx.handle, s.ctypes.data, sp, s.nbytes))
    ctx._check(ctx.lib.qwh_download(ctx.handle, d.ctypes.data, dp, d.nbytes))
    ctx.matrix_release(m)
    return sh.quantized_payload(sh.o.Q4, s, d)


def norms():
    rng = np.random.default_rng(5)
    c = TINY
    out = {}
    for layer in range(c["layers"]):
        out[(T_ATTN_NORM, layer)] = (1 + 0.1 * rng.standard_normal(c["hidden"])).astype(np.float32)
        out[(T_FFN_NORM, layer)] = (1 + 0.1 * rng.standard_normal(c["hidden"])).astype(np.float32)
        # Stored as f16 and bf16 in the shard: values exact in those formats.
        out[(T_Q_NORM, layer)] = (1 + 0.1 * rng.standard_normal(c["head_dim"])).astype(np.float16).astype(np.float32)
        kb = (1 + 0.1 * rng.standard_normal(c["head_dim"])).astype(np.float32)
        out[(T_K_NORM, layer)] = ((kb.view(np.uint32) >> 16) << 16).view(np.float32)
    out[(T_FINAL_NORM, 0)] = (1 + 0.1 * rng.standard_normal(c["hidden"])).astype(np.float32)
    return out


def build_shards(ctx, with_output=True, fmt=qa.FORMAT_Q4):
    c = TINY
    qw, kvw = c["heads"] * c["head_dim"], c["kv_heads"] * c["head_dim"]
    nv = norms()
    glob = [dict(kind=sh.KIND_DECODER_EMBED_TOKENS, layer=0, format=fmt, dims=(c["vocab"], c["hidden"]),
                 payload=planes(ctx, c["vocab"], c["hidden"], 1, fmt)),
            dict(kind=sh.KIND_DECODER_FINAL_NORM, layer=0, format=sh.F32, dims=(c["hidden"],),
                 payload=nv[(T_FINAL_NORM, 0)].tobytes())]
    if with_output:
        glob.append(dict(kind=sh.KIND_DECODER_OUTPUT, layer=0, format=fmt, dims=(c["vocab"], c["hidden"]),
                         payload=planes(ctx, c["vocab"], c["hidden"], 2, fmt)))
    per_layer = []
    for layer in range(c["layers"]):
        sb = 16 + 16 * layer
        shapes = {33: (qw, c["hidden"], sb), 34: (kvw, c["hidden"], sb + 1), 35: (kvw, c["hidden"], sb + 2),
                  36: (c["hidden"], qw, sb + 3), 41: (c["ffn"], c["hidden"], sb + 4),
                  42: (c["ffn"], c["hidden"], sb + 5), 43: (c["hidden"], c["ffn"], sb + 6)}
        tensors = [dict(kind=k, layer=layer + 1, format=fmt, dims=(r, cc), payload=planes(ctx, r, cc, st, fmt))
                   for k, (r, cc, st) in shapes.items()]
        tensors += [
            dict(kind=39, layer=layer + 1, format=sh.F32, dims=(c["hidden"],), payload=nv[(T_ATTN_NORM, layer)].tobytes()),
            dict(kind=40, layer=layer + 1, format=sh.F32, dims=(c["hidden"],), payload=nv[(T_FFN_NORM, layer)].tobytes()),
            dict(kind=37, layer=layer + 1, format=sh.F16, dims=(c["head_dim"],),
                 payload=nv[(T_Q_NORM, layer)].astype(np.float16).tobytes()),
            dict(kind=38, layer=layer + 1, format=sh.BF16, dims=(c["head_dim"],),
                 payload=(nv[(T_K_NORM, layer)].view(np.uint32) >> 16).astype(np.uint16).tobytes()),
        ]
        per_layer.append(tensors)
    # Shard 1: the model-wide tensors and layer 1; shard 2: layer 2.
    return [sh.build(glob + per_layer[0]), sh.build(per_layer[1])], nv


def reference_decoder(ctx, nv, tied=False, fmt=qa.FORMAT_Q4):
    d = qa.Decoder(ctx, batch=2, **TINY)
    d.init_synthetic(SEED, fmt)
    for (kind, layer), values in nv.items():
        d.set_vector(kind, layer, values)
    if tied:
        m = ctx.matrix_synthetic(fmt, TINY["vocab"], TINY["hidden"], SEED, 1, 0.02)
        d.set_matrix(T_LM_HEAD, 0, m)
        ctx.matrix_release(m)
    return d


def config_bin(tied: bool) -> bytes:
    """A config.bin for the TINY decoder (model_config.zig layout; the audio
    fields are the 0.6B model's, with the projector width the hidden size)."""
    c = TINY
    tokens = {k: 990 + i for i, k in enumerate(mc.TOKENS)}
    return mc.pack(dict(mc.CONFIG_0P6B, text_hidden_size=c["hidden"], audio_output_dim=c["hidden"],
                        text_layers=c["layers"], text_attention_heads=c["heads"],
                        text_key_value_heads=c["kv_heads"], text_head_dim=c["head_dim"], text_ffn_dim=c["ffn"],
                        vocab_size=c["vocab"], max_positions=c["max_positions"], flags=1 if tied else 0,
                        **tokens))


@pytest.mark.parametrize("tied,fmt", [(False, qa.FORMAT_Q4), (True, qa.FORMAT_Q4), (False, qa.FORMAT_F16),
                                      (True, qa.FORMAT_F16)])
def test_decoder_bound_from_shards(ctx, tied, fmt):
    blobs, nv = build_shards(ctx, with_output=not tied, fmt=fmt)
    for blob in blobs:
        assert sh.parse(blob)[0] == sh.OK
    ref = reference_decoder(ctx, nv, tied, fmt)
    # The model as a loader sees it: config.bin, then the shards.
    status, reason, model = qa.config_parse(config_bin(tied))
    assert (status, reason) == (0, 0)
    dims = qa.config_decoder(model)
    assert {k: dims[k] for k in TINY if k not in ("eps", "theta")} == {k: v for k, v in TINY.items()
                                                                     if k not in ("eps", "theta")}
    dec = qa.Decoder(ctx, batch=2, **dims)
    try:
        counts = []
        for blob in blobs:
            shard = ctx.shard_load(blob)
            counts.append(dec.bind_shard(shard, output_tied=bool(model.flags & 1)))
            ctx.shard_release(shard)   # the decoder holds copies
        assert counts == [3 + 11, 11]   # embed, final norm, output (or tied), and 11 per layer
        for d in (ref, dec):
            d.prefill_random(0, 5, SEED)
            d.prefill_random(1, 11, SEED)
        tokens = [7, 300]
        ref.forward(tokens, True)
        dec.forward(tokens, True)
        for b in range(2):
            assert np.array_equal(ref.logits(b), dec.logits(b)), b
        assert np.array_equal(ref.generate([1, 2], 12), dec.generate([1, 2], 12))
    finally:
        ref.close()
        dec.close()
