// config.bin (model_config.zig): the 160-byte architecture configuration of
// a converted model, parsed and validated on the host (no device), and the
// decoder dimensions it implies.
//
// model_config.parse (model_config.zig:354-360) and Config.validate (:260-327)
// are followed check by check and in the same order. The reference's ABI maps
// the configuration's errors to invalid_argument (or truncated / bad_magic /
// bad_version, wasm/abi.zig:90-146); `reason` reports which check failed, as
// the value list of qwhip.h's QWH_CONFIG_* (model_config.zig:89-106 order).
#include <cmath>
#include <cstring>

#include "common.h"

namespace {

constexpr uint32_t kFieldMax = 1u << 24;       // model_config.zig:26
constexpr uint32_t kLayerMax = 512;            // :27
constexpr uint32_t kVocabMax = 1u << 21;       // :28
constexpr uint32_t kDecodeTokensMax = 8192;    // :29
constexpr uint32_t kMelBins = 128;             // mel.zig:50
constexpr uint64_t kCapacityFrames = 480000 / 160;  // mel.zig:56-58
constexpr uint32_t kKnownFlags = QWH_CONFIG_OUTPUT_TIED;

bool in_range(uint32_t v) { return v != 0 && v <= kFieldMax; }
bool layers_ok(uint32_t v) { return v != 0 && v <= kLayerMax; }

// (n - 1) / 2 + 1 three times: the convolution stack's stride-2 steps.
uint64_t after_convolutions(uint64_t n) {
    for (int i = 0; i < 3; ++i) n = (n - 1) / 2 + 1;
    return n;
}

uint32_t validate(const qwh_model_config &c) {
    if (std::memcmp(c.magic, "QWCFG001", 8) != 0) return QWH_CONFIG_BAD_MAGIC;
    if (c.format_version != 1) return QWH_CONFIG_BAD_VERSION;
    if ((c.flags & ~kKnownFlags) != 0 || c.reserved[0] || c.reserved[1] || c.reserved[2])
        return QWH_CONFIG_RESERVED_NOT_EMPTY;
    if (c.architecture != 1) return QWH_CONFIG_UNKNOWN_ARCHITECTURE;  // qwen3_asr

    for (uint32_t v : {c.audio_d_model, c.audio_ffn_dim, c.audio_downsample_hidden_size, c.audio_output_dim,
                       c.text_hidden_size, c.text_ffn_dim, c.text_head_dim})
        if (!in_range(v)) return QWH_CONFIG_INVALID_DIMENSION;
    if (!layers_ok(c.audio_layers) || !layers_ok(c.text_layers)) return QWH_CONFIG_INVALID_DIMENSION;

    if (c.mel_bins != kMelBins) return QWH_CONFIG_INVALID_MEL_GEOMETRY;
    if (c.audio_attention_heads == 0 || c.audio_d_model % c.audio_attention_heads != 0)
        return QWH_CONFIG_INVALID_HEAD_GEOMETRY;
    const uint32_t audio_head_dim = c.audio_d_model / c.audio_attention_heads;
    if (audio_head_dim < 2 || audio_head_dim % 2 != 0) return QWH_CONFIG_INVALID_HEAD_GEOMETRY;
    if (c.text_attention_heads == 0 || c.text_key_value_heads == 0 ||
        c.text_attention_heads % c.text_key_value_heads != 0)
        return QWH_CONFIG_INVALID_HEAD_GEOMETRY;
    // The query width (heads * head_dim) may differ from the hidden size.
    if (c.text_head_dim < 2 || c.text_head_dim % 2 != 0) return QWH_CONFIG_INVALID_HEAD_GEOMETRY;
    if (c.text_hidden_size != c.audio_output_dim) return QWH_CONFIG_INVALID_DIMENSION;

    if (c.audio_n_window == 0) return QWH_CONFIG_INVALID_CHUNK_GEOMETRY;
    const uint64_t chunk = (uint64_t)c.audio_n_window * 2;
    if (chunk > kCapacityFrames) return QWH_CONFIG_INVALID_CHUNK_GEOMETRY;
    if (c.audio_n_window_infer % chunk != 0) return QWH_CONFIG_INVALID_CHUNK_GEOMETRY;
    if (c.audio_max_position_steps < after_convolutions(chunk)) return QWH_CONFIG_INVALID_CHUNK_GEOMETRY;
    if (c.mel_bins % 8 != 0) return QWH_CONFIG_INVALID_MEL_GEOMETRY;

    if (c.vocab_size == 0 || c.vocab_size > kVocabMax) return QWH_CONFIG_INVALID_DIMENSION;
    if (!in_range(c.max_positions)) return QWH_CONFIG_INVALID_DIMENSION;
    if (c.max_decode_tokens == 0 || c.max_decode_tokens > kDecodeTokensMax) return QWH_CONFIG_INVALID_DIMENSION;

    if (!std::isfinite(c.audio_layer_norm_eps) || !std::isfinite(c.text_rms_norm_eps))
        return QWH_CONFIG_INVALID_EPSILON;
    if (!(c.audio_layer_norm_eps > 0.0f) || !(c.text_rms_norm_eps > 0.0f)) return QWH_CONFIG_INVALID_EPSILON;
    if (!std::isfinite(c.rope_theta) || !(c.rope_theta > 1.0f)) return QWH_CONFIG_INVALID_ROPE_THETA;

    for (uint32_t t : {c.token_audio_start, c.token_audio_end, c.token_audio_pad, c.token_im_start, c.token_im_end,
                       c.token_endoftext, c.token_asr_text, c.token_eos_primary, c.token_eos_secondary, c.token_pad})
        if (t >= c.vocab_size) return QWH_CONFIG_INVALID_TOKEN_ID;
    return QWH_CONFIG_OK;
}

int32_t status_of(uint32_t reason) {
    switch (reason) {
    case QWH_CONFIG_OK: return QWH_OK;
    case QWH_CONFIG_BAD_MAGIC: return QWH_E_BAD_MAGIC;
    case QWH_CONFIG_BAD_VERSION: return QWH_E_BAD_VERSION;
    case QWH_CONFIG_TRUNCATED: return QWH_E_TRUNCATED;
    default: return QWH_E_INVALID_ARGUMENT;
    }
}

}  // namespace

static_assert(sizeof(qwh_model_config) == 160, "config.bin is 160 bytes (model_config.zig:362-374)");

extern "C" {

int32_t qwh_config_parse(const void *bytes, uint64_t len, qwh_model_config *out, uint32_t *reason) {
    uint32_t r;
    qwh_model_config c;
    if (!bytes) return QWH_E_INVALID_ARGUMENT;
    if (len != sizeof(qwh_model_config)) {
        r = QWH_CONFIG_TRUNCATED;
    } else if (((uintptr_t)bytes & 3u) != 0) {
        r = QWH_CONFIG_MISALIGNED;
    } else {
        std::memcpy(&c, bytes, sizeof c);
        r = validate(c);
    }
    if (reason) *reason = r;
    if (r == QWH_CONFIG_OK && out) *out = c;
    return status_of(r);
}

int32_t qwh_config_decoder(const qwh_model_config *model, qwh_decoder_config *out) {
    if (!model || !out) return QWH_E_INVALID_ARGUMENT;
    out->hidden = model->text_hidden_size;
    out->layers = model->text_layers;
    out->heads = model->text_attention_heads;
    out->kv_heads = model->text_key_value_heads;
    out->head_dim = model->text_head_dim;
    out->ffn = model->text_ffn_dim;
    out->vocab = model->vocab_size;
    out->max_positions = model->max_positions;
    out->eps = model->text_rms_norm_eps;
    out->theta = model->rope_theta;
    return QWH_OK;
}

}  // extern "C"
