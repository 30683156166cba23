/*
 * qwref: CPU oracle for the quantized decoder hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference
 * implementation (mattneel/qwenscriber, Zig) that the HIP backend is checked
 * against. Only tests/, __graft_entry__.smoke() and the cpu_baseline leg of
 * bench.py may load it, and only as the checker or the timed CPU baseline --
 * never as the thing measured or shipped.
 *
 * Every function cites the reference file:line it restates. Arithmetic is
 * IEEE f32 with one rounding per operation, in the reference's order; the
 * library is compiled with -ffp-contract=off and without fast-math so that
 * no multiply-add is fused behind the restatement's back.
 *
 * Pinning (what checks each part beyond retyping it):
 *   f16 codec        half_float.zig:47-77 known answers + comparison against
 *                    numpy's float16 casts (every f16 pattern widened; a sweep
 *                    of f32 values, ties included, narrowed) in the tests.
 *   quantize/pack    selftest.zig:294 golden quant_hash 0xf247917b05691fd1,
 *                    quant.zig:527-554 exact values, plane offsets :423-448.
 *   dequant / dot    kernels.zig:932-971 (ones row -> 56.0), f64 brute force.
 *   linear           kernels.zig:840-930, f64 brute force on small shapes.
 *   linear f16 / f32 kernels.zig:932-948 (ones -> 64), numpy's f16 widening
 *                    bit for bit, f64 brute force over every finite f16 class.
 *   embedding row    decoder.zig:378-420 known answers (f32 exact, f16 within
 *                    1e-3, q4 within 0.2), numpy's widening bit for bit.
 *   attention (q8)   kernels.zig:769-836 (q8 vs f32 within 0.05), closed forms
 *                    (one-hot query on identical keys = mean of V), f64 brute force.
 *   glue             math.zig:174-214 known answers, RoPE norm invariance.
 *   audio glue       math.zig:134-171 erf / gelu known answers (C library erf
 *                    at double precision), kernels.zig:1162-1171 addBias values,
 *                    f64 numpy layer norm and windowed attention brute force,
 *                    kernels.zig:1043-1078 windowed-attention known answers.
 *   audio layer      composition of the pinned parts (no reference-held vectors).
 *   audio front end  kernels.zig:973-1041 convolution known answers,
 *                    model.zig:1136-1170 sinusoid known answers,
 *                    model_config.zig:431 (3000 frames -> 375 steps), f64
 *                    brute force of the convolution, and the composition
 *                    (chunks, flatten, projection, positions) against float64.
 *   decoder step     composition of the pinned parts (q4 / q5 / q8 / f16 / f32 weights,
 *                    f32 / q8 cache, non-unit norm weights) checked against an
 *                    independent float64 restatement; no reference-held
 *                    vectors exist for random weights (parity unpinned end to
 *                    end beyond that composition).
 *   transcendentals  expf/powf/sinf/cosf are glibc's, not Zig compiler_rt's:
 *                    parity unpinned at the last ulp (tolerance-pinned only).
 */
#ifndef QWREF_H
#define QWREF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype.zig:17-108 format ids, quant.zig:47-63 group constants. */
enum { QWREF_F32 = 0, QWREF_F16 = 1, QWREF_Q4 = 16, QWREF_Q5 = 17, QWREF_Q8 = 18 };
enum { QWREF_GROUP = 64 };

typedef struct {
    uint64_t scales_offset_bytes;
    uint64_t scales_len_bytes;
    uint64_t data_offset_bytes;
    uint64_t data_len_bytes;
    uint64_t total_len_bytes;
    uint32_t group_count;
    uint32_t groups_per_row;
} qwref_layout;

/* Status values follow src/wasm/abi.zig:50-73. */
enum {
    QWREF_OK = 0,
    QWREF_INVALID_ARGUMENT = -1,
    QWREF_UNSUPPORTED = -3,
    QWREF_SHAPE_MISMATCH = -7,
    QWREF_LIMIT_EXCEEDED = -9,
};

/* ---- L0 numerics ---------------------------------------------------- */
uint16_t qwref_to_f16(float value);
float qwref_from_f16(uint16_t bits);
uint16_t qwref_to_bf16(float value);
float qwref_from_bf16(uint16_t bits);

int32_t qwref_bias(int32_t format);
int32_t qwref_data_bytes_per_group(int32_t format);
int32_t qwref_plane_layout(int32_t format, uint32_t rows, uint32_t cols, uint64_t base,
                           uint64_t alignment, qwref_layout *out);
uint64_t qwref_plane_bytes(int32_t format, uint32_t positions, uint32_t cols);

void qwref_quantize_row(int32_t format, const float *values, uint32_t cols, uint8_t *scales_out,
                        uint8_t *data_out);
void qwref_quantize_rows(int32_t format, const float *values, uint32_t rows, uint32_t cols,
                         uint8_t *scales_out, uint8_t *data_out);
void qwref_dequantize_row(int32_t format, const uint8_t *row_scales, const uint8_t *row_data,
                          float *out, uint32_t cols);
float qwref_dot_row(int32_t format, const uint8_t *row_scales, const uint8_t *row_data,
                    const float *x, uint32_t cols);
uint64_t qwref_quant_hash(void);
uint64_t qwref_fnv1a64(const uint8_t *bytes, uint64_t len, uint64_t state);

/* ---- L1 kernels ------------------------------------------------------- */
float qwref_dot_f32(const float *left, const float *right, uint32_t len);
int32_t qwref_linear_quantized(float *out, const float *x, int32_t format, const uint8_t *scales,
                               uint64_t scales_len, const uint8_t *data, uint64_t data_len,
                               uint32_t rows, uint32_t cols, uint32_t tokens);
int32_t qwref_linear_f32(float *out, const float *x, const float *weights, uint32_t rows,
                         uint32_t cols, uint32_t tokens);
int32_t qwref_linear_f16(float *out, const float *x, const uint16_t *weights, uint32_t rows,
                         uint32_t cols, uint32_t tokens);
int32_t qwref_embedding_row(int32_t format, const uint8_t *scales, const uint8_t *data, uint32_t rows,
                            uint32_t cols, uint32_t row, float *out);
void qwref_add_in_place(float *x, const float *y, uint32_t len);
void qwref_silu_mul(float *out, const float *gate, const float *up, uint32_t len);
float qwref_silu(float x);
void qwref_softmax_in_place(float *row, uint32_t len);
void qwref_rms_norm(float *x, const float *weight, uint32_t width, uint32_t tokens, float eps);
float qwref_inverse_frequency(uint32_t index, uint32_t head_dim, float theta);
void qwref_build_rope_tables(float *cos_table, float *sin_table, uint32_t half, float theta,
                             uint32_t max_positions, uint32_t stride);
void qwref_rope_in_place(float *rotated, const uint32_t *positions, uint32_t tokens,
                         uint32_t heads, uint32_t head_dim, const float *cos_table,
                         const float *sin_table, uint32_t table_stride);
int32_t qwref_decode_attention_step(float *out, const float *query, const float *keys,
                                    const float *values, uint32_t cached, uint32_t heads,
                                    uint32_t kv_heads, uint32_t head_dim);
int32_t qwref_decode_attention_step_q8(float *out, const float *query, const uint8_t *k_scales,
                                       const uint8_t *k_codes, const uint8_t *v_scales,
                                       const uint8_t *v_codes, uint32_t cached, uint32_t heads,
                                       uint32_t kv_heads, uint32_t head_dim);
uint32_t qwref_argmax(const float *logits, uint32_t count);

/* Audio tower glue (kernels.zig:210-271, :429-484; math.zig:46-66, :99-116). */
float qwref_erf(float x);
float qwref_gelu(float x);
void qwref_gelu_in_place(float *x, uint64_t len);
int32_t qwref_add_bias(float *x, const float *bias, uint32_t rows, uint32_t tokens);
void qwref_layer_norm(float *x, const float *weight, const float *bias, uint32_t width, uint32_t tokens,
                      float eps);
int32_t qwref_audio_attention_window(float *out, uint32_t out_stride, const float *q, uint32_t q_stride,
                                     const float *k, uint32_t k_stride, const float *v, uint32_t v_stride,
                                     uint32_t window_start, uint32_t window_length, uint32_t heads,
                                     uint32_t head_dim);

/* Audio convolution front end (kernels.zig:302-427; model.zig:509-644,
 * :751-763; model_config.zig:84-90). Weights are f16 bits [out][in][3][3]. */
uint32_t qwref_post_convolution_steps(uint32_t frames);
int32_t qwref_conv3x3s2_gelu(float *out, const float *input, const uint16_t *weights, const float *bias,
                             uint32_t out_channels, uint32_t in_channels, uint32_t in_height, uint32_t in_width);
void qwref_add_sinusoidal_position(float *row, uint32_t step, uint32_t channels);

/* ---- synthetic inputs (test-input specification, not reference code) --- */
uint32_t qwref_mulberry32_at(uint32_t seed, uint64_t draw);
float qwref_normal_at(uint32_t seed, uint32_t stream, uint64_t index);
void qwref_fill_normal(float *out, uint64_t count, uint32_t seed, uint32_t stream, float scale);
uint32_t qwref_stream_base(uint32_t seed, uint32_t stream);

/* ---- L2 decoder (decoder.zig restatement) ------------------------------ */
typedef struct {
    uint32_t hidden;
    uint32_t layers;
    uint32_t heads;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t ffn;
    uint32_t vocab;
    uint32_t max_positions;
    float eps;
    float theta;
} qwref_decoder_config;

typedef struct qwref_decoder qwref_decoder;

/* Cache formats: model_config.zig:44-68 CacheFormat values. */
enum { QWREF_CACHE_F32 = 0, QWREF_CACHE_Q8 = 1 };
/* Norm weight vectors a decoder holds (decoder.zig:165-172, :180-193,
 * :259-265, :277-284); the values are the library's tensor kinds. */
enum {
    QWREF_VEC_ATTENTION_NORM = 16,
    QWREF_VEC_Q_NORM = 17,
    QWREF_VEC_K_NORM = 18,
    QWREF_VEC_FFN_NORM = 19,
    QWREF_VEC_FINAL_NORM = 20,
};

/* Builds a decoder whose every linear is q4, from the synthetic generator
 * (seed, stream ids documented in qwref.c), norm weights all 1.0, q8 cache. */
qwref_decoder *qwref_decoder_create_synthetic(const qwref_decoder_config *config, uint32_t seed,
                                              uint32_t batch);
/* The same synthetic values with every linear (and the embedding) quantized
 * to `weight_format` (q4, q5 or q8) or stored as f32 / f16 (rounded to
 * nearest even), and the key/value cache in `cache_format`. NULL for an
 * unknown format. */
qwref_decoder *qwref_decoder_create_synthetic_as(const qwref_decoder_config *config, uint32_t seed,
                                                 uint32_t batch, int32_t weight_format,
                                                 int32_t cache_format);
void qwref_decoder_destroy(qwref_decoder *decoder);
/* Replaces one norm weight vector (kind QWREF_VEC_*, layer ignored for the
 * final norm); count must be hidden (attention, ffn, final) or head_dim
 * (q, k). */
int32_t qwref_decoder_set_vector(qwref_decoder *decoder, uint32_t kind, uint32_t layer,
                                 const float *values, uint32_t count);
/* Fills positions [0, count) of every layer's cache of sequence `seq` from
 * the generator (N(0,1) rows, stored as f32 or as quantizeRow(.q8)), and
 * sets its position. */
int32_t qwref_decoder_prefill_random(qwref_decoder *decoder, uint32_t seq, uint32_t count);
int32_t qwref_decoder_forward(qwref_decoder *decoder, uint32_t seq, uint32_t token,
                              int32_t want_logits);
int32_t qwref_decoder_forward_row(qwref_decoder *decoder, uint32_t seq, uint32_t token, const float *audio_row,
                                  int32_t want_logits);
const float *qwref_decoder_logits(qwref_decoder *decoder, uint32_t seq);
uint32_t qwref_decoder_position(qwref_decoder *decoder, uint32_t seq);
int32_t qwref_decoder_step(qwref_decoder *decoder, uint32_t seq, uint32_t token,
                           uint32_t *next_token);
/* FNV-1a-64 over every weight plane in upload order (embed, per layer q k v o
 * gate up down, lm_head; scales then data). */
uint64_t qwref_decoder_weights_hash(qwref_decoder *decoder);
uint64_t qwref_decoder_cache_hash(qwref_decoder *decoder, uint32_t seq);
/* One cache row: q8 key scales, key codes, value scales, value codes (f32:
 * key row, value row); returns the bytes written, 0 on a bad argument. */
uint64_t qwref_decoder_cache_row(qwref_decoder *decoder, uint32_t seq, uint32_t layer, uint32_t position,
                                 uint8_t *out, uint64_t capacity);
/* Test plumbing: store a row in the cache_row layout (0, or
 * QWREF_INVALID_ARGUMENT), and set a sequence's position. */
int32_t qwref_decoder_set_cache_row(qwref_decoder *decoder, uint32_t seq, uint32_t layer, uint32_t position,
                                    const uint8_t *row, uint64_t len);
int32_t qwref_decoder_set_position(qwref_decoder *decoder, uint32_t seq, uint32_t position);
uint32_t qwref_synthetic_start_token(uint32_t seed, uint32_t seq, uint32_t vocab);

void qwref_set_threads(int32_t threads);

#ifdef __cplusplus
}
#endif
#endif
