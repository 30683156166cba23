/*
 * qwhip.h -- C ABI of the MI355X (gfx950) backend for Qwenscriber's quantized
 * decoder hot path.
 *
 * The reference (mattneel/qwenscriber) runs this path in Zig on the CPU
 * (src/core/qwen3_asr/kernels.zig, decoder.zig) and in WGSL on WebGPU
 * (the gpu/shaders directory, driven by packages/qwenscriber/src/gpu/text_decoder.ts).
 * This library is one more backend behind the same operator surface: the
 * caller keeps the reference's packed weight planes (quant.zig:8-41: groups of
 * 64, one f16 scale per group in a scale plane, biased unsigned codes in a
 * data plane) and its q8 key/value cache layout (decoder.zig:58-106), and
 * calls these entry points instead of the Zig kernels.
 *
 * Conventions (mirroring src/wasm/abi.zig and kernels.zig):
 *   - every entry point returns an int32 status; 0 is success, failures are
 *     the negative values of abi.zig:50-73 (QWH_E_*), plus QWH_E_DEVICE for a
 *     HIP runtime failure, which has no counterpart in the reference;
 *   - shapes are checked before any device work, and a mismatch returns
 *     QWH_E_SHAPE_MISMATCH, as kernels.zig's Error.ShapeMismatch does;
 *   - plain pointers and sizes only. `*_dev` pointers are device addresses
 *     (from qwh_alloc or any HIP allocation on the context's device); other
 *     pointers are host memory;
 *   - a context owns one device and one stream. Calls are stream ordered and
 *     return without waiting, except where a host output is produced (those
 *     synchronize the stream). A context is used by one host thread at a time.
 */
#ifndef QWHIP_H
#define QWHIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QWH_ABI_VERSION 0x00010000 /* major << 16 | minor, as abi.zig's abi_version */

/* Status codes: src/wasm/abi.zig:50-73. */
#define QWH_OK 0
#define QWH_E_INVALID_ARGUMENT (-1)
#define QWH_E_OUT_OF_MEMORY (-2)
#define QWH_E_UNSUPPORTED (-3)
#define QWH_E_SHAPE_MISMATCH (-7)
#define QWH_E_INVALID_STATE (-8)
#define QWH_E_LIMIT_EXCEEDED (-9)
#define QWH_E_NOT_FOUND (-10)
/* Shard statuses (abi.zig:58-63, :72-77; mapping abi.zig:90-146). */
#define QWH_E_BAD_MAGIC (-4)
#define QWH_E_BAD_VERSION (-5)
#define QWH_E_CHECKSUM_MISMATCH (-6)
#define QWH_E_TRUNCATED (-11)
#define QWH_E_UNSUPPORTED_MODEL (-13)
/* A HIP runtime error. Not in the reference (it has no device runtime). */
#define QWH_E_DEVICE (-64)

/* Format ids: src/core/dtype.zig:17-108 (on-disk values, never renumbered).
 * Matrices hold f32, f16 (kernels.zig:160-166 Matrix) or a quantized format. */
#define QWH_FORMAT_F32 0
#define QWH_FORMAT_F16 1
#define QWH_FORMAT_Q4 16
#define QWH_FORMAT_Q5 17
#define QWH_FORMAT_Q8 18

/* Quantization group: src/core/quant.zig:49. */
#define QWH_GROUP_SIZE 64

typedef struct qwh_ctx qwh_ctx;

/* ---------------------------------------------------------------------- */
/* Context, memory, timing                                                 */
/* ---------------------------------------------------------------------- */

/* Replaces wasm/exports.zig `qw_abi_version`. */
int32_t qwh_abi_version(void);
/* Human-readable name of a status code (static storage). */
const char *qwh_status_string(int32_t status);
/* Opens device `device_index` with a stream of its own. No reference
 * counterpart: the Zig core has no device (it replaces model arena setup,
 * wasm/model.zig:197-204, for the device side). */
int32_t qwh_create(uint32_t device_index, qwh_ctx **out);
int32_t qwh_destroy(qwh_ctx *ctx);
/* Waits for all work queued on the context's stream. */
int32_t qwh_sync(qwh_ctx *ctx);
/* Text of the last failure on this context (empty when none). */
const char *qwh_last_error(qwh_ctx *ctx);
/* Number of compute units of the context's device. */
int32_t qwh_device_cus(qwh_ctx *ctx, uint32_t *out);

/* Device buffers for callers without a HIP allocator of their own (a Zig or
 * JavaScript host). Copies are stream ordered; downloads synchronize. */
int32_t qwh_alloc(qwh_ctx *ctx, uint64_t bytes, void **out_dev);
int32_t qwh_free(qwh_ctx *ctx, void *dev);
int32_t qwh_upload(qwh_ctx *ctx, void *dst_dev, const void *src, uint64_t bytes);
int32_t qwh_download(qwh_ctx *ctx, void *dst, const void *src_dev, uint64_t bytes);
int32_t qwh_memset(qwh_ctx *ctx, void *dst_dev, int32_t value, uint64_t bytes);

/* Stream-ordered timing: records event `slot` (0..255) on the context stream;
 * qwh_event_elapsed synchronizes on `end` and returns milliseconds. */
int32_t qwh_event_record(qwh_ctx *ctx, uint32_t slot);
int32_t qwh_event_elapsed(qwh_ctx *ctx, uint32_t start, uint32_t end, float *out_ms);

/* Roofline calibration, no reference counterpart: a plain streaming read of
 * `bytes` at src_dev (16-byte aligned, a multiple of 16) with the GEMVs' load
 * form, by cus * blocks_per_cu (1..8) workgroups, each writing one word to
 * sink_dev. The bench times it over the same buffers as a GEMV to give the
 * achievable read bandwidth next to the HBM peak. */
int32_t qwh_stream_read(qwh_ctx *ctx, const void *src_dev, uint64_t bytes, uint32_t blocks_per_cu,
                        uint32_t *sink_dev);

/* ---------------------------------------------------------------------- */
/* Weight matrices (kernels.zig Matrix, quant.zig planeLayout)             */
/* ---------------------------------------------------------------------- */

/* Uploads a rows x cols quantized matrix given as the two planes
 * quant.planeLayout (quant.zig:144-176) describes: `scales` is rows *
 * cols/64 f16 values (little endian, groups row major), `data` the packed
 * codes. The row count must agree with the scale plane as Matrix.rows
 * derives it (kernels.zig:170-178). Replaces Binding.matrix
 * (model.zig:92-114) for the device. For QWH_FORMAT_F32 / QWH_FORMAT_F16
 * (the Matrix .f32 / .f16 arms, kernels.zig:161-166) there is no scale plane
 * (scales may be NULL, scales_len must be 0) and `data` holds the rows * cols
 * elements row major (f16 as little-endian bit patterns), any cols >= 1. */
int32_t qwh_matrix_upload(qwh_ctx *ctx, int32_t format, uint32_t rows, uint32_t cols,
                          const uint8_t *scales, uint64_t scales_len, const uint8_t *data,
                          uint64_t data_len, uint64_t *out_matrix);
/* Borrows planes already resident on the device (for example a whole .qw
 * shard uploaded at once): the caller keeps them alive until release, as the
 * reference's Matrix borrows shard bytes (wasm/model.zig:28-42). Quantized
 * data planes 16-byte aligned; f32 / f16 elements aligned to their size
 * (model.zig:79-90), scales_dev ignored. */
int32_t qwh_matrix_wrap(qwh_ctx *ctx, int32_t format, uint32_t rows, uint32_t cols,
                        const void *scales_dev, const void *data_dev, uint64_t *out_matrix);
/* A matrix whose values are f32(N(0,1)) * value_scale from the synthetic
 * generator (seed, stream), quantized on the device bit-exactly as
 * quant.quantizeRow (f16: rounded to nearest even, half_float.zig:12-16;
 * f32: as generated). For benchmarks and tests with random-init weights. */
int32_t qwh_matrix_synthetic(qwh_ctx *ctx, int32_t format, uint32_t rows, uint32_t cols,
                             uint32_t seed, uint32_t stream, float value_scale,
                             uint64_t *out_matrix);
/* Device addresses of a matrix's two planes (no scale plane, NULL, for f32
 * and f16). */
int32_t qwh_matrix_planes(qwh_ctx *ctx, uint64_t matrix, void **scales_dev, void **data_dev);
int32_t qwh_matrix_release(qwh_ctx *ctx, uint64_t matrix);

/* ---------------------------------------------------------------------- */
/* `.qw` weight shards (container.zig)                                     */
/* ---------------------------------------------------------------------- */

/* One index entry as stored on disk (container.zig:103-125 Entry, 40 bytes):
 * kind is a container.TensorKind value (:337-381), layer 0 for tensors of
 * no layer, 1..text_layers for decoder layers, 1024 + i for audio layers;
 * format is a dtype.Format value (0 f32, 1 f16, 2 bf16, 16 q4, 17 q5, 18 q8);
 * offset_bytes is relative to the payload. */
typedef struct qwh_tensor_entry {
    uint16_t kind;
    uint16_t layer;
    uint8_t format;
    uint8_t rank;
    uint16_t reserved;
    uint32_t dims[4];
    uint64_t offset_bytes;
    uint64_t len_bytes;
} qwh_tensor_entry;

/* container.File.parse (container.zig:175-217) on the host, no device
 * needed: the header, then every entry in order (known format, shape, exact
 * length), sorted by (layer, kind), ranges in order, 16-byte aligned and
 * inside the payload. Statuses as the reference ABI maps File.parse's errors:
 * QWH_E_BAD_MAGIC, QWH_E_BAD_VERSION, QWH_E_TRUNCATED, QWH_E_SHAPE_MISMATCH
 * (shape or byte length), QWH_E_UNSUPPORTED_MODEL (unknown format),
 * QWH_E_INVALID_ARGUMENT (index not sorted, ranges overlapping or
 * misaligned). */
int32_t qwh_shard_validate(const void *bytes, uint64_t len, uint32_t *tensor_count);
/* File.verifyChecksum (container.zig:283-290): the header's checksum against
 * the low 32 bits of FNV-1a 64 over the payload; QWH_E_CHECKSUM_MISMATCH. */
int32_t qwh_shard_verify_checksum(const void *bytes, uint64_t len);
/* File.find (container.zig:226-236): the entry of (kind, layer), or
 * QWH_E_NOT_FOUND. */
int32_t qwh_shard_find(const void *bytes, uint64_t len, uint16_t kind, uint16_t layer,
                       qwh_tensor_entry *out);
/* Validates a shard and copies its payload to the device once; the bytes may
 * be freed afterwards. */
int32_t qwh_shard_load(qwh_ctx *ctx, const void *bytes, uint64_t len, uint64_t *out_shard);
/* File.tensorBytes (container.zig:238-243) on the device: the address of a
 * tensor inside the loaded payload (and its entry, when `entry` is set). */
int32_t qwh_shard_tensor(qwh_ctx *ctx, uint64_t shard, uint16_t kind, uint16_t layer, void **dev,
                         qwh_tensor_entry *entry);
/* File.quantizedPlanes (container.zig:248-266) as a matrix handle that
 * borrows the two planes inside the loaded payload (no copy). f32 / f16
 * tensors of rank 2 become matrices over their elements in place, as
 * Binding.matrix makes them (model.zig:92-96); other element tensors (bf16,
 * vectors) return QWH_E_NOT_FOUND, as quantizedPlanes returns null. */
int32_t qwh_shard_matrix(qwh_ctx *ctx, uint64_t shard, uint16_t kind, uint16_t layer,
                         uint64_t *out_matrix);
/* Frees the device payload; QWH_E_INVALID_STATE while a matrix borrows from
 * it. */
int32_t qwh_shard_release(qwh_ctx *ctx, uint64_t shard);

/* kernels.zig:182-206 Matrix.apply / :118-158 linearQuantized:
 * out[tokens][rows] = W[rows][cols] * x[tokens][cols], f32 in, f32 out.
 * `cols` must equal the matrix's column count. Formats q4 and q8 at any
 * shape; q5 (the WebGPU decoder's format, passes.ts:63-67) for cols <= 6144
 * with an 8-byte aligned data plane below 4 GiB; f32 and f16
 * (linearF32 / linearF16, :54-112) for cols <= 40956; else
 * QWH_E_UNSUPPORTED. */
int32_t qwh_linear(qwh_ctx *ctx, uint64_t matrix, const float *x_dev, uint32_t cols,
                   uint32_t tokens, float *out_dev);
/* qwh_linear in two halves, for callers that apply several matrices to the
 * same activations (decoder.zig:174-176 applies q, k and v to one `normed`
 * row): qwh_activation_prepare encodes x once into `prepared_dev` (at least
 * qwh_activation_bytes(cols, tokens) bytes), qwh_linear_prepared multiplies a
 * q4 matrix by it. The results equal qwh_linear's. */
int32_t qwh_activation_bytes(uint32_t cols, uint32_t tokens, uint64_t *out_bytes);
int32_t qwh_activation_prepare(qwh_ctx *ctx, const float *x_dev, uint32_t cols, uint32_t tokens,
                               void *prepared_dev);
int32_t qwh_linear_prepared(qwh_ctx *ctx, uint64_t matrix, const void *prepared_dev,
                            uint32_t tokens, float *out_dev);
/* The same product with bf16 activations (the prefill / audio-token GEMM of
 * the reference's tokens > 1 path, kernels.zig:118-158 with tokens = M). The
 * reference widens each bf16 to f32 (half_float.zig:42-45) before the dot.
 * q4, q5 and q8 matrices (q5 with an 8-byte, q8 with a 16-byte aligned data
 * plane). */
int32_t qwh_linear_bf16(qwh_ctx *ctx, uint64_t matrix, const uint16_t *x_dev, uint32_t cols,
                        uint32_t tokens, float *out_dev);

/* ---------------------------------------------------------------------- */
/* Device quantization (quant.zig:197-288)                                 */
/* ---------------------------------------------------------------------- */

/* quant.quantizeRow applied to `rows` rows of `cols` f32 values on the
 * device, bit exact: scales_dev receives rows*cols/64 f16 values, data_dev the
 * packed codes. Formats q4, q5, q8. */
int32_t qwh_quantize_rows(qwh_ctx *ctx, int32_t format, const float *values_dev, uint32_t rows,
                          uint32_t cols, uint8_t *scales_dev, uint8_t *data_dev);
/* Fills `count` f32 values with the synthetic generator (value i of stream
 * `stream` under `seed`, times value_scale). */
int32_t qwh_synth_normal(qwh_ctx *ctx, uint32_t seed, uint32_t stream, uint64_t count,
                         float value_scale, float *out_dev);

/* ---------------------------------------------------------------------- */
/* q8 key/value cache and decode attention                                 */
/* ---------------------------------------------------------------------- */

/* kernels.zig:697-767 decodeAttentionStepQ8, with device pointers:
 * query_dev [heads*head_dim] f32, the four planes of one layer's cache
 * (decoder.zig:58-65 cachePlane: k/v scales [positions][kv_heads*head_dim/64]
 * f16, k/v codes [positions][kv_heads*head_dim] u8), `cached` positions read.
 * `batch` independent sequences are laid out back to back: query and out
 * advance by heads*head_dim floats, the planes by `plane_stride_bytes`
 * (scales) and `code_stride_bytes` (codes) per sequence. Any head_dim that
 * is a multiple of 64 up to 1024 and any heads / kv_heads ratio (head_dim
 * 64 / 128 / 256 with ratios up to 8, or 2 at 256, run the split-range
 * kernels; the other shapes a one-workgroup-per-head kernel); a wider head
 * returns QWH_E_UNSUPPORTED. */
int32_t qwh_decode_attention_q8(qwh_ctx *ctx, float *out_dev, const float *query_dev,
                                const uint8_t *k_scales_dev, const uint8_t *k_codes_dev,
                                const uint8_t *v_scales_dev, const uint8_t *v_codes_dev,
                                uint32_t cached, uint32_t heads, uint32_t kv_heads,
                                uint32_t head_dim, uint32_t batch, uint64_t scale_stride_bytes,
                                uint64_t code_stride_bytes);

/* qwh_decode_attention_q8 without any allocation. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, hosts that forbid it). The
 * range records live in a static device array of 8 MiB per GPU, resolved at
 * qwh_create; inputs needing more (about batch * kv_heads * ranges records of
 * (heads/kv_heads) * (head_dim + 4) floats) return QWH_E_LIMIT_EXCEEDED.
 * Calls on one GPU share that array: calls that overlap on one GPU (two
 * contexts' streams) race. Results equal qwh_decode_attention_q8's. */
int32_t qwh_decode_attention_q8_noalloc(qwh_ctx *ctx, float *out_dev, const float *query_dev,
                                        const uint8_t *k_scales_dev, const uint8_t *k_codes_dev,
                                        const uint8_t *v_scales_dev, const uint8_t *v_codes_dev, uint32_t cached,
                                        uint32_t heads, uint32_t kv_heads, uint32_t head_dim, uint32_t batch,
                                        uint64_t scale_stride_bytes, uint64_t code_stride_bytes);

/* kernels.zig:572-627 decodeAttentionStep over an f32 cache (the reference's
 * default cache, model_config.zig:44-68): keys_dev / values_dev are
 * [positions][kv_heads*head_dim] f32 (decoder.zig:77-83), `cached` positions
 * read; `batch` sequences back to back, query and out advancing by
 * heads*head_dim floats, keys and values by `stride_bytes`. Any head_dim up
 * to 1024 and any heads / kv_heads ratio (split-range kernels for head_dim
 * 64 / 128 / 256, a one-workgroup-per-head kernel otherwise); a wider head
 * returns QWH_E_UNSUPPORTED. */
int32_t qwh_decode_attention_f32(qwh_ctx *ctx, float *out_dev, const float *query_dev, const float *keys_dev,
                                 const float *values_dev, uint32_t cached, uint32_t heads, uint32_t kv_heads,
                                 uint32_t head_dim, uint32_t batch, uint64_t stride_bytes);

/* decoder.zig:68-106 appendCacheRow (q8): quantizes one key row and one value
 * row of kv_width f32 values into row `position` of a layer's planes, bit
 * exact with quant.quantizeRow(.q8). */
int32_t qwh_kv_append_q8(qwh_ctx *ctx, const float *key_dev, const float *value_dev,
                         uint32_t kv_width, uint32_t position, uint8_t *k_scales_dev,
                         uint8_t *k_codes_dev, uint8_t *v_scales_dev, uint8_t *v_codes_dev);

/* decoder.zig:290-301 argmaxLogits for `rows` rows of `count` logits
 * (rows back to back): ids_dev[r] = the index of the row's largest value, the
 * lowest such index among equal maxima; a row whose first value is NaN, or
 * with no value above -FLT_MAX, gives 0 (the reference's scan keeps index 0
 * unless a later value compares greater). The decoder step's argmax. */
int32_t qwh_argmax_rows(qwh_ctx *ctx, const float *logits_dev, uint32_t rows, uint32_t count, uint32_t *ids_dev);

/* ---------------------------------------------------------------------- */
/* Audio tower and projector (model.zig:646-735)                           */
/* ---------------------------------------------------------------------- */

/* kernels.zig:259-271 layerNormInto (math.zig:99-116 per row): out = (x -
 * mean) / sqrt(variance + eps) * weight + bias over `tokens` rows of `width`
 * floats. out may equal x (kernels.zig:242-255 layerNorm in place). */
int32_t qwh_layer_norm(qwh_ctx *ctx, float *out_dev, const float *x_dev, const float *weight_dev,
                       const float *bias_dev, uint32_t width, uint32_t tokens, float eps);

/* kernels.zig:210-218 addBias: x[t][r] += bias[r] for `tokens` rows of `rows`. */
int32_t qwh_add_bias(qwh_ctx *ctx, float *x_dev, const float *bias_dev, uint32_t rows, uint32_t tokens);

/* math.zig:63-66 gelu over `count` values in place (model.zig:719, :868). */
int32_t qwh_gelu(qwh_ctx *ctx, float *x_dev, uint64_t count);

/* kernels.zig:429-484 audioAttentionWindow: non-causal attention of the steps
 * [window_start, window_start + window_length) over the same steps, per head;
 * row r of q / k / v / out starts at ptr + r * stride (floats). The scores
 * scratch the reference takes is internal. Built for head_dim 32, 64 and
 * 128; strides multiples of 4 and buffers 16-byte aligned. */
int32_t qwh_audio_attention_window(qwh_ctx *ctx, float *out_dev, uint32_t out_stride, const float *q_dev,
                                   uint32_t q_stride, const float *k_dev, uint32_t k_stride, const float *v_dev,
                                   uint32_t v_stride, uint32_t window_start, uint32_t window_length,
                                   uint32_t heads, uint32_t head_dim);

/* model.zig:792-822 runWindowedAttention: every window of `window_steps`
 * steps from step 0 (the last one ragged) in one launch; q / k / v share one
 * row stride, as the reference's packed q | k | v buffer does. */
int32_t qwh_audio_attention(qwh_ctx *ctx, float *out_dev, uint32_t out_stride, const float *q_dev,
                            const float *k_dev, const float *v_dev, uint32_t qkv_stride, uint32_t steps,
                            uint32_t window_steps, uint32_t heads, uint32_t head_dim);

/* One audio tower layer's weights (model.zig AudioLayer): matrix handles of
 * the context, and device f32 vectors. */
typedef struct {
    uint64_t q, k, v, o;       /* d_model x d_model */
    uint64_t ffn_in;           /* ffn_dim x d_model */
    uint64_t ffn_out;          /* d_model x ffn_dim */
    const float *q_bias, *k_bias, *v_bias, *o_bias, *ffn_in_bias, *ffn_out_bias;
    const float *attention_norm_weight, *attention_norm_bias;
    const float *final_norm_weight, *final_norm_bias;
} qwh_audio_layer_weights;

/* model.zig:656-693, one iteration of runAudioTower's layer loop over the
 * residual stream encoder[steps][d_model] (updated in place): LayerNorm,
 * q / k / v + bias, windowed attention, o + bias + residual, LayerNorm,
 * ffn_in + bias, GELU, ffn_out + bias + residual. Scratch is the context's. */
int32_t qwh_audio_layer(qwh_ctx *ctx, const qwh_audio_layer_weights *weights, float *encoder_dev,
                        uint32_t steps, uint32_t d_model, uint32_t heads, uint32_t ffn_dim,
                        uint32_t window_steps, float eps);

/* kernels.zig:302-427 conv3x3Stride2Gelu over `batch` independent images:
 * in [batch][in_channels][in_height][in_width] f32, weights
 * [out_channels][in_channels][3][3] f16 bits (the checkpoint's layout), bias
 * [out_channels]; out [batch][out_channels][(h-1)/2+1][(w-1)/2+1] =
 * gelu(bias + the 3x3, stride 2, padding 1 convolution). */
int32_t qwh_conv3x3s2_gelu(qwh_ctx *ctx, float *out_dev, const float *in_dev, const uint16_t *weights_dev,
                           const float *bias_dev, uint32_t batch, uint32_t out_channels, uint32_t in_channels,
                           uint32_t in_height, uint32_t in_width);

/* The audio tower's convolution front end (model.zig AudioModel conv1..3,
 * conv_out): device f16-bit conv weights [downsample][in][3][3] (conv1 has
 * one input channel), f32 biases, and conv_out as a matrix handle of
 * d_model x downsample * bins, bins = mel_bins after three halvings. */
typedef struct {
    const uint16_t *conv1_weight, *conv2_weight, *conv3_weight;
    const float *conv1_bias, *conv2_bias, *conv3_bias;
    uint64_t conv_out;
} qwh_audio_frontend_weights;

/* model.zig:509-644 convolveAndPack + projectConvStep: the log-mel
 * spectrogram [mel_bins][frames] (f32, device) in chunks of 2 * n_window
 * frames (the last zero filled), three conv3x3Stride2Gelu stages, each valid
 * time step flattened channel-major over the remaining frequency bins,
 * projected by conv_out, plus the sinusoidal position of the step within its
 * chunk (model.zig:751-763). Writes the packed encoder rows [steps][d_model]
 * (steps = model_config.zig:226-238 for `frames`) to encoder_dev, which holds
 * encoder_rows rows (else QWH_E_LIMIT_EXCEEDED); steps_out receives steps.
 * Scratch is the context's. */
int32_t qwh_audio_frontend(qwh_ctx *ctx, const qwh_audio_frontend_weights *weights, const float *log_mel_dev,
                           uint32_t mel_bins, uint32_t frames, uint32_t n_window, uint32_t downsample,
                           uint32_t d_model, float *encoder_dev, uint32_t encoder_rows, uint32_t *steps_out);

/* model.zig:707-735 runProjector: out[steps][hidden] = W_out gelu(W_in x +
 * b_in) + b_out, W_in d_model x d_model, W_out hidden x d_model. */
int32_t qwh_audio_projector(qwh_ctx *ctx, uint64_t in_matrix, const float *in_bias_dev,
                            uint64_t out_matrix, const float *out_bias_dev, const float *encoder_dev,
                            uint32_t steps, float *out_dev);

/* ---------------------------------------------------------------------- */
/* Decoder step (decoder.zig:133-339)                                      */
/* ---------------------------------------------------------------------- */

/* model_config.zig:110-258, the fields the decoder step reads. */
typedef struct {
    uint32_t hidden;        /* text_hidden_size */
    uint32_t layers;        /* text_layers */
    uint32_t heads;         /* text_attention_heads */
    uint32_t kv_heads;      /* text_key_value_heads */
    uint32_t head_dim;      /* text_head_dim */
    uint32_t ffn;           /* text_ffn_dim */
    uint32_t vocab;         /* vocab_size */
    uint32_t max_positions; /* max_positions (model.zig:62 caps it at 8192) */
    float eps;              /* text_rms_norm_eps */
    float theta;            /* rope_theta */
} qwh_decoder_config;

/* Tensor kinds a decoder binds (layout.zig decoder tensors). */
#define QWH_T_EMBED 0
#define QWH_T_Q 1
#define QWH_T_K 2
#define QWH_T_V 3
#define QWH_T_O 4
#define QWH_T_GATE 5
#define QWH_T_UP 6
#define QWH_T_DOWN 7
#define QWH_T_LM_HEAD 8
#define QWH_T_ATTN_NORM 16
#define QWH_T_Q_NORM 17
#define QWH_T_K_NORM 18
#define QWH_T_FFN_NORM 19
#define QWH_T_FINAL_NORM 20

typedef struct qwh_decoder qwh_decoder;

/* Key/value cache formats: model_config.zig:44-68 CacheFormat values. */
#define QWH_CACHE_F32 0u
#define QWH_CACHE_Q8 1u

/* Creates a decoder for `batch` independent sequences, each with its own q8
 * key/value cache of config->max_positions positions (decoder.zig:58-65
 * layout, per layer [scales][codes]). RoPE tables are built on the host by
 * kernels.zig:534-564 (buildRopeTables) semantics, as model.zig:400-407 does.
 * Every matrix starts as a zero q4 matrix; bind them with
 * qwh_decoder_set_matrix, qwh_decoder_bind_shard or qwh_decoder_init_synthetic. */
int32_t qwh_decoder_create(qwh_ctx *ctx, const qwh_decoder_config *config, uint32_t batch,
                           qwh_decoder **out);
/* qwh_decoder_create with the cache in `cache_format` (model.zig's
 * cache_format, chosen by transcribe.zig's --cache f32|q8):
 * QWH_CACHE_F32 keeps per layer [max_positions][kv_heads * head_dim] f32 keys
 * and values (decoder.zig:77-83) and attends with decodeAttentionStep
 * (kernels.zig:572-627); QWH_CACHE_Q8 is qwh_decoder_create's cache. */
int32_t qwh_decoder_create_cache(qwh_ctx *ctx, const qwh_decoder_config *config, uint32_t batch,
                                 uint32_t cache_format, qwh_decoder **out);
int32_t qwh_decoder_destroy(qwh_decoder *decoder);
/* Binds a matrix (QWH_T_EMBED..QWH_T_LM_HEAD) in q4, q5, q8, f16 or f32:
 * each matrix is applied in its own format, as Matrix.apply applies whatever
 * storage it holds (kernels.zig:182-206), and an f32 / f16 embedding gives
 * its rows as embeddingRow does (decoder.zig:346-360). f32 / f16 rows of up
 * to 40956 values. The decoder copies the planes into
 * its own blocks: q / k / v into one fused row block and gate / up into one
 * block with their rows interleaved (gate row j, then up row j). A fused
 * block holds one format, so binding a member in another format re-creates
 * the block (zeroed) and its other members are bound again after it.
 * Layer is ignored for EMBED and LM_HEAD. */
int32_t qwh_decoder_set_matrix(qwh_decoder *decoder, uint32_t kind, uint32_t layer,
                               uint64_t matrix);
/* Binds an f32 norm weight vector (host pointer, copied). */
int32_t qwh_decoder_set_vector(qwh_decoder *decoder, uint32_t kind, uint32_t layer,
                               const float *values, uint32_t count);
/* Binds every decoder tensor a loaded `.qw` shard holds (qwh_shard_load):
 * container.TensorKind 30..43 (container.zig:367-380) at layer 0 (embedding,
 * final norm, output projection) and layers 1..layers (the decoder's layer
 * L - 1); other kinds (audio tower, projector) are skipped. Matrices may be
 * q4, q5, q8, or f16 / f32 tensors of rank 2 (the converter writes one
 * format for all, layout.zig:49-53, f16 for --quantization none)
 * and are copied (the shard may be released afterwards); norm vectors
 * may be f32, f16 or bf16 and are widened to f32. With
 * QWH_BIND_OUTPUT_TIED (config.bin flags bit 0, model_config.zig) the
 * embedding is also bound as the output projection. A model split over
 * several shards takes one call per shard. `bound` receives the number of
 * slots filled. */
#define QWH_BIND_OUTPUT_TIED 1u
int32_t qwh_decoder_bind_shard(qwh_decoder *decoder, uint64_t shard, uint32_t flags, uint32_t *bound);
/* Binds every matrix from the synthetic generator: each linear q4 with
 * values f32(N(0,1)) * 0.02, stream ids as the oracle's synthetic model.
 * Norm weights are left as they are (1.0 unless set). */
int32_t qwh_decoder_init_synthetic(qwh_decoder *decoder, uint32_t seed);
/* The same synthetic values quantized to `format` (q4, q5 or q8), or stored
 * as f32 / f16 (rounded to nearest even), for every matrix, the embedding
 * included. */
int32_t qwh_decoder_init_synthetic_format(qwh_decoder *decoder, uint32_t seed, int32_t format);
/* decoder.zig:109-121 reset: zeroes every cache and sets positions to 0. */
int32_t qwh_decoder_reset(qwh_decoder *decoder);
/* Fills positions [0, count) of sequence `seq`'s caches with quantizeRow(.q8)
 * of synthetic N(0,1) rows and sets its position to `count`. */
int32_t qwh_decoder_prefill_random(qwh_decoder *decoder, uint32_t seq, uint32_t count,
                                   uint32_t seed);
/* Device addresses of sequence `seq`, layer `layer`'s cache planes (with an
 * f32 cache the scale planes are NULL and the code planes hold the f32
 * rows). */
int32_t qwh_decoder_cache_planes(qwh_decoder *decoder, uint32_t seq, uint32_t layer,
                                 void **k_scales, void **k_codes, void **v_scales,
                                 void **v_codes);
int32_t qwh_decoder_position(qwh_decoder *decoder, uint32_t seq, uint32_t *out);
int32_t qwh_decoder_set_position(qwh_decoder *decoder, uint32_t seq, uint32_t position);
/* decoder.zig:133-287 forwardToken for every sequence at once: tokens[b] is
 * sequence b's token. With want_logits the logits stay on the device. */
int32_t qwh_decoder_forward(qwh_decoder *decoder, const uint32_t *tokens, int32_t want_logits);
/* decoder.zig:133-150 forwardToken with audio_row: for every sequence whose
 * row_mask byte is nonzero (every sequence when row_mask is null), row b of
 * rows_dev (batch x hidden f32, device) replaces the token's embedding --
 * the projected audio features spliced into a placeholder position, as
 * decoder.zig:308-333 prefill does. Other sequences embed tokens[b]. Every
 * sequence advances one position; logits are kept when want_logits. */
int32_t qwh_decoder_forward_rows(qwh_decoder *decoder, const uint32_t *tokens, const float *rows_dev,
                                 const uint8_t *row_mask, int32_t want_logits);
/* decoder.zig:308-333 Decoder.prefill for sequence `seq`: its `count`
 * prompt tokens (host array) at positions position(seq) .. + count - 1, each
 * audio_pad_token taking the next of audio_steps projected audio rows
 * (audio_rows_dev: audio_steps x hidden f32, device) in place of its
 * embedding; every position's key and value rows are appended to the cache,
 * the sequence's position advances by count, and *next_token receives the
 * greedy token after the prompt (argmaxLogits of its last position; those
 * logits stay on the device). An empty prompt, or audio pads that do not
 * match audio_steps, give QWH_E_SHAPE_MISMATCH (the reference's
 * UnexpectedShape / PromptMismatch). The positions are processed together,
 * in chunks of 256: each layer's products run over all of them, their cache
 * rows are appended, then each attends to the cache rows up to its own.
 * Layer matrices without a matrix-core form run their per-token GEMV once
 * over a chunk's rows (f32 / f16, q5 / q8, and q4 rows its fused GEMV
 * takes). Where some matrix has neither (a q4 row of an odd number of
 * 32-value slices the fused GEMV does not take), a batch-1 decoder runs the
 * prompt through its step one position at a time; a larger batch gets
 * QWH_E_UNSUPPORTED (the step would advance its other sequences). Tokens
 * past the vocabulary give QWH_E_SHAPE_MISMATCH and a prompt past
 * max_positions QWH_E_LIMIT_EXCEEDED; every check runs before any position,
 * so a refused prompt leaves the sequence as it was. */
int32_t qwh_decoder_prefill(qwh_decoder *decoder, uint32_t seq, const uint32_t *tokens, uint32_t count,
                            uint32_t audio_pad_token, const float *audio_rows_dev, uint32_t audio_steps,
                            uint32_t *next_token);
/* decoder.zig:336-339 step: forwardToken then argmaxLogits (:290-301, first
 * maximum wins) for every sequence; next_tokens receives batch ids. */
int32_t qwh_decoder_step(qwh_decoder *decoder, const uint32_t *tokens, uint32_t *next_tokens);
/* Runs `steps` greedy steps, feeding each argmax back, entirely on the device
 * (the step graph is replayed without host round trips); ids_out receives
 * steps x batch ids, step major. */
int32_t qwh_decoder_generate(qwh_decoder *decoder, const uint32_t *tokens, uint32_t steps,
                             uint32_t *ids_out);
/* Greedy decoding with the stop rules of wasm/model.zig:423-451 decodeStep
 * (and :495-499 endsSequence), entirely on the device: tokens[b] is sequence
 * b's next token (the prediction of its last prompt position). Per
 * sequence, while it has not finished: a token among stop_tokens (at most 3:
 * token_eos_primary, token_eos_secondary, token_endoftext) ends it and is not
 * emitted; otherwise the token is emitted, and once max_tokens ids are out
 * the sequence ends without another prediction; otherwise step() predicts
 * the next token. A finished sequence is frozen (its position no longer
 * advances) while the others continue. ids_out receives max_tokens x batch
 * ids, step major (rows past a sequence's count are 0); counts_out[b] the
 * number of ids sequence b emitted. Positions advance by the forwards each
 * sequence ran. */
int32_t qwh_decoder_generate_until(qwh_decoder *decoder, const uint32_t *tokens, uint32_t max_tokens,
                                   const uint32_t *stop_tokens, uint32_t stop_count, uint32_t *ids_out,
                                   uint32_t *counts_out);
/* Copies sequence `seq`'s last logits (vocab f32) to the host. */
int32_t qwh_decoder_logits(qwh_decoder *decoder, uint32_t seq, float *out, uint32_t count);

/* ---------------------------------------------------------------------- */
/* config.bin (model_config.zig)                                           */
/* ---------------------------------------------------------------------- */

/* model_config.Config (model_config.zig:110-190), the 160-byte on-disk
 * layout, little endian. */
typedef struct qwh_model_config {
    char magic[8]; /* "QWCFG001" */
    uint32_t format_version;
    uint32_t architecture; /* 1 = qwen3_asr */
    uint32_t audio_d_model, audio_layers, audio_attention_heads, audio_ffn_dim;
    uint32_t audio_downsample_hidden_size, audio_n_window, audio_n_window_infer;
    uint32_t audio_max_position_steps, audio_output_dim, mel_bins;
    float audio_layer_norm_eps;
    uint32_t text_hidden_size, text_layers, text_attention_heads, text_key_value_heads;
    uint32_t text_head_dim, text_ffn_dim, vocab_size;
    float text_rms_norm_eps, rope_theta;
    uint32_t max_positions, max_decode_tokens;
    uint32_t token_audio_start, token_audio_end, token_audio_pad, token_im_start, token_im_end;
    uint32_t token_endoftext, token_asr_text, token_eos_primary, token_eos_secondary, token_pad;
    uint32_t flags;       /* bit 0: output projection tied to the embedding */
    uint32_t reserved[3]; /* zero */
} qwh_model_config;

#define QWH_CONFIG_OUTPUT_TIED 1u
/* Which check rejected a configuration: model_config.Error in its declared
 * order (model_config.zig:89-106). */
#define QWH_CONFIG_OK 0u
#define QWH_CONFIG_BAD_MAGIC 1u
#define QWH_CONFIG_BAD_VERSION 2u
#define QWH_CONFIG_TRUNCATED 3u
#define QWH_CONFIG_RESERVED_NOT_EMPTY 4u
#define QWH_CONFIG_UNKNOWN_ARCHITECTURE 5u
#define QWH_CONFIG_INVALID_DIMENSION 6u
#define QWH_CONFIG_INVALID_HEAD_GEOMETRY 7u
#define QWH_CONFIG_INVALID_MEL_GEOMETRY 8u
#define QWH_CONFIG_INVALID_TOKEN_ID 9u
#define QWH_CONFIG_INVALID_EPSILON 10u
#define QWH_CONFIG_INVALID_ROPE_THETA 11u
#define QWH_CONFIG_INVALID_CHUNK_GEOMETRY 12u
#define QWH_CONFIG_MISALIGNED 13u

/* model_config.parse (model_config.zig:354-360) + Config.validate
 * (:260-327) on the host, no device: exactly 160 bytes, 4-byte aligned, then
 * every check in the reference's order. Status as the reference ABI maps
 * the errors (QWH_E_TRUNCATED, QWH_E_BAD_MAGIC, QWH_E_BAD_VERSION, else
 * QWH_E_INVALID_ARGUMENT); `reason` (optional) receives the QWH_CONFIG_*
 * value; `out` (optional) the configuration when it is valid. */
int32_t qwh_config_parse(const void *bytes, uint64_t len, qwh_model_config *out, uint32_t *reason);
/* The decoder dimensions of a configuration (text_* fields, vocab_size,
 * max_positions, rope_theta), for qwh_decoder_create. */
int32_t qwh_config_decoder(const qwh_model_config *model, qwh_decoder_config *out);

#ifdef __cplusplus
}
#endif
#endif
