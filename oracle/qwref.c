/*
 * qwref.c -- CPU oracle for the quantized decoder hot path. TEST INFRASTRUCTURE.
 *
 * A plain-C restatement of mattneel/qwenscriber's Zig CPU kernels, used only
 * as the checker of the HIP backend and as the timed single-core CPU
 * baseline. Each function names the reference lines it follows. Build flags
 * (oracle/Makefile): -O3 -ffp-contract=off, no fast-math, so every f32
 * operation rounds once, in the order written, as Zig's strict float mode does.
 */
#include "qwref.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 1;

void qwref_set_threads(int32_t threads) { g_threads = threads > 0 ? threads : 1; }

/* ------------------------------------------------------------------------ */
/* half_float.zig:14-45                                                      */
/* ------------------------------------------------------------------------ */

static uint32_t f32_bits(float v) {
    uint32_t b;
    memcpy(&b, &v, 4);
    return b;
}

static float bits_f32(uint32_t b) {
    float v;
    memcpy(&v, &b, 4);
    return v;
}

/* Shift right, rounding the discarded bits to nearest, ties to even. */
static uint32_t round_shift_right(uint32_t value, uint32_t shift) {
    uint32_t kept = value >> shift;
    uint32_t remainder = value & ((1u << shift) - 1u);
    uint32_t halfway = 1u << (shift - 1u);
    if (remainder > halfway) return kept + 1u;
    if (remainder < halfway) return kept;
    return kept + (kept & 1u);
}

/* half_float.zig:14-17 `toF16`: @floatCast f32->f16, round to nearest even,
 * overflow to infinity. Written out in bits because the host compiler has no
 * f16 type; tests compare it exhaustively with numpy's float16 cast. */
uint16_t qwref_to_f16(float value) {
    uint32_t bits = f32_bits(value);
    uint32_t sign = (bits >> 16) & 0x8000u;
    int32_t exponent = (int32_t)((bits >> 23) & 0xffu);
    uint32_t mantissa = bits & 0x7fffffu;
    if (exponent == 0xff) return (uint16_t)(sign | 0x7c00u | (mantissa ? 0x200u : 0u));
    int32_t half_exponent = exponent - 127 + 15;
    if (half_exponent >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (half_exponent <= 0) {
        if (half_exponent < -10) return (uint16_t)sign;
        mantissa |= 0x800000u;
        /* A subnormal result that rounds up into the smallest normal carries
         * into the exponent field by itself. */
        return (uint16_t)(sign | round_shift_right(mantissa, (uint32_t)(14 - half_exponent)));
    }
    uint32_t rounded = round_shift_right(mantissa, 13);
    /* A mantissa that rounds up to 0x400 carries into the exponent; the sum
     * below does that, and reaches 0x7c00 (infinity) from the largest finite. */
    return (uint16_t)(sign | (((uint32_t)half_exponent << 10) + rounded));
}

/* half_float.zig:20-23 `fromF16`: exact widening. */
float qwref_from_f16(uint16_t bits) {
    uint32_t sign = (uint32_t)(bits & 0x8000u) << 16;
    uint32_t exponent = (bits >> 10) & 0x1fu;
    uint32_t mantissa = bits & 0x3ffu;
    if (exponent == 0) {
        if (mantissa == 0) return bits_f32(sign);
        /* Subnormal: value = mantissa * 2^-24, exact in f32. */
        float magnitude = (float)mantissa * 5.9604644775390625e-08f;
        return sign ? -magnitude : magnitude;
    }
    if (exponent == 31) return bits_f32(sign | 0x7f800000u | (mantissa << 13));
    return bits_f32(sign | ((exponent - 15u + 127u) << 23) | (mantissa << 13));
}

/* half_float.zig:30-39 `toBf16`. */
uint16_t qwref_to_bf16(float value) {
    uint32_t bits = f32_bits(value);
    if ((bits & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((bits >> 16) | 0x0040u);
    uint32_t round_bias = 0x7fffu + ((bits >> 16) & 1u);
    return (uint16_t)((bits + round_bias) >> 16);
}

/* half_float.zig:42-45 `fromBf16`. */
float qwref_from_bf16(uint16_t bits) { return bits_f32((uint32_t)bits << 16); }

/* ------------------------------------------------------------------------ */
/* quant.zig                                                                 */
/* ------------------------------------------------------------------------ */

/* quant.zig:111-118 */
int32_t qwref_bias(int32_t format) {
    switch (format) {
    case QWREF_Q4: return 8;
    case QWREF_Q5: return 16;
    case QWREF_Q8: return 128;
    default: return 0;
    }
}

/* quant.zig:52-59, :102-109 */
int32_t qwref_data_bytes_per_group(int32_t format) {
    switch (format) {
    case QWREF_Q4: return 32;
    case QWREF_Q5: return 40;
    case QWREF_Q8: return 64;
    default: return 0;
    }
}

static uint64_t align_forward(uint64_t value, uint64_t alignment) {
    return (value + alignment - 1u) / alignment * alignment;
}

/* quant.zig:144-176 `planeLayout`. */
int32_t qwref_plane_layout(int32_t format, uint32_t rows, uint32_t cols, uint64_t base,
                           uint64_t alignment, qwref_layout *out) {
    if (format != QWREF_Q4 && format != QWREF_Q5 && format != QWREF_Q8) return QWREF_UNSUPPORTED;
    if (alignment < 4 || alignment % 4 != 0) return QWREF_INVALID_ARGUMENT;
    if (cols % QWREF_GROUP != 0) return QWREF_SHAPE_MISMATCH;
    uint32_t group_count = rows == 0 ? 0 : rows * (cols / QWREF_GROUP);
    uint64_t scales_len = (uint64_t)group_count * 2u;
    uint64_t data_len = (uint64_t)group_count * (uint64_t)qwref_data_bytes_per_group(format);
    uint64_t scales_offset = align_forward(base, alignment) - base;
    uint64_t data_start = base + scales_offset + scales_len;
    uint64_t data_offset = align_forward(data_start, alignment) - base;
    out->scales_offset_bytes = scales_offset;
    out->scales_len_bytes = scales_len;
    out->data_offset_bytes = data_offset;
    out->data_len_bytes = data_len;
    out->total_len_bytes = data_offset + data_len;
    out->group_count = group_count;
    out->groups_per_row = cols / QWREF_GROUP;
    return QWREF_OK;
}

/* quant.zig:183-191 `planeBytes`. */
uint64_t qwref_plane_bytes(int32_t format, uint32_t positions, uint32_t cols) {
    uint64_t groups = (uint64_t)positions * ((uint64_t)cols / QWREF_GROUP);
    if (format == QWREF_F32) return (uint64_t)positions * cols * 4u;
    return groups * 2u + groups * (uint64_t)qwref_data_bytes_per_group(format);
}

/* quant.zig:280-288 `quantizeOne`: round half away from zero in f32 via
 * floor(x + 0.5) / ceil(x - 0.5), then clamp. */
static int32_t quantize_one(float value, float stored_scale, int32_t min_code, int32_t max_code) {
    if (stored_scale == 0.0f) return 0;
    float scaled = value / stored_scale;
    float rounded = scaled >= 0.0f ? floorf(scaled + 0.5f) : ceilf(scaled - 0.5f);
    if (rounded <= (float)min_code) return min_code;
    if (rounded >= (float)max_code) return max_code;
    return (int32_t)rounded;
}

/* quant.zig:229-278 `quantizeGroup`. */
static void quantize_group(int32_t format, const float *values, float stored_scale, uint8_t *codes) {
    int32_t shift = qwref_bias(format);
    int32_t min_code = -shift;
    int32_t max_code = shift - 1;
    switch (format) {
    case QWREF_Q4:
        memset(codes, 0, 32);
        for (int index = 0; index < QWREF_GROUP; ++index) {
            uint8_t u = (uint8_t)(quantize_one(values[index], stored_scale, min_code, max_code) + shift);
            if (index % 2 == 0) codes[index / 2] |= u;
            else codes[index / 2] |= (uint8_t)(u << 4);
        }
        break;
    case QWREF_Q5:
        memset(codes, 0, 40);
        for (int index = 0; index < QWREF_GROUP; ++index) {
            uint8_t u = (uint8_t)(quantize_one(values[index], stored_scale, min_code, max_code) + shift);
            uint8_t low = u & 0x0f;
            if (index % 2 == 0) codes[index / 2] |= low;
            else codes[index / 2] |= (uint8_t)(low << 4);
            if (u & 0x10) codes[32 + index / 8] |= (uint8_t)(1u << (index % 8));
        }
        break;
    case QWREF_Q8:
        for (int index = 0; index < QWREF_GROUP; ++index)
            codes[index] = (uint8_t)(quantize_one(values[index], stored_scale, min_code, max_code) + shift);
        break;
    default: break;
    }
}

/* quant.zig:197-227 `quantizeRow`: scale = f16(max_abs / bias), codes against
 * the stored scale. */
void qwref_quantize_row(int32_t format, const float *values, uint32_t cols, uint8_t *scales_out,
                        uint8_t *data_out) {
    uint32_t group_count = cols / QWREF_GROUP;
    int32_t data_bytes = qwref_data_bytes_per_group(format);
    for (uint32_t g = 0; g < group_count; ++g) {
        const float *group = values + (size_t)g * QWREF_GROUP;
        float max_abs = 0.0f;
        for (int i = 0; i < QWREF_GROUP; ++i) {
            float a = fabsf(group[i]);
            /* @max(max_abs, |v|) */
            max_abs = a > max_abs ? a : max_abs;
        }
        uint16_t scale_bits = qwref_to_f16(max_abs / (float)qwref_bias(format));
        scales_out[g * 2] = (uint8_t)(scale_bits & 0xff);
        scales_out[g * 2 + 1] = (uint8_t)(scale_bits >> 8);
        float stored_scale = qwref_from_f16(scale_bits);
        quantize_group(format, group, stored_scale, data_out + (size_t)g * data_bytes);
    }
}

/* quantizeRow applied row by row, as the converter does (convert.zig:763-791):
 * groups stay row-major across both planes. */
void qwref_quantize_rows(int32_t format, const float *values, uint32_t rows, uint32_t cols,
                         uint8_t *scales_out, uint8_t *data_out) {
    uint32_t gpr = cols / QWREF_GROUP;
    int32_t data_bytes = qwref_data_bytes_per_group(format);
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int64_t r = 0; r < (int64_t)rows; ++r) {
        qwref_quantize_row(format, values + (size_t)r * cols, cols, scales_out + (size_t)r * gpr * 2,
                           data_out + (size_t)r * gpr * data_bytes);
    }
}

static uint16_t read_f16_le(const uint8_t *bytes, size_t group) {
    return (uint16_t)(bytes[group * 2] | ((uint16_t)bytes[group * 2 + 1] << 8));
}

/* quant.zig:315-345 `dequantizeGroup`: f32(u - bias), then *= scale. */
static void dequantize_group(int32_t format, const uint8_t *codes, float scale, float *out) {
    int32_t shift = qwref_bias(format);
    switch (format) {
    case QWREF_Q4:
        for (int i = 0; i < QWREF_GROUP; ++i) {
            uint8_t byte = codes[i / 2];
            uint8_t nibble = (i % 2 == 0) ? (byte & 0x0f) : (byte >> 4);
            out[i] = (float)((int32_t)nibble - shift);
        }
        break;
    case QWREF_Q5:
        for (int i = 0; i < QWREF_GROUP; ++i) {
            uint8_t byte = codes[i / 2];
            uint32_t low = (i % 2 == 0) ? (byte & 0x0fu) : (uint32_t)(byte >> 4);
            uint32_t high = (codes[32 + i / 8] >> (i % 8)) & 1u;
            out[i] = (float)((int32_t)(low | (high << 4)) - shift);
        }
        break;
    case QWREF_Q8:
        for (int i = 0; i < QWREF_GROUP; ++i) out[i] = (float)((int32_t)codes[i] - shift);
        break;
    default: break;
    }
    for (int i = 0; i < QWREF_GROUP; ++i) out[i] *= scale;
}

/* quant.zig:348-364 `dequantizeRow`. */
void qwref_dequantize_row(int32_t format, const uint8_t *row_scales, const uint8_t *row_data,
                          float *out, uint32_t cols) {
    int32_t data_bytes = qwref_data_bytes_per_group(format);
    for (uint32_t g = 0; g < cols / QWREF_GROUP; ++g) {
        float scale = qwref_from_f16(read_f16_le(row_scales, g));
        dequantize_group(format, row_data + (size_t)g * data_bytes, scale, out + (size_t)g * QWREF_GROUP);
    }
}

/* quant.zig:370-391 `dotRow`: one scalar f32 accumulator, group by group. */
float qwref_dot_row(int32_t format, const uint8_t *row_scales, const uint8_t *row_data,
                    const float *x, uint32_t cols) {
    int32_t data_bytes = qwref_data_bytes_per_group(format);
    float accumulator = 0.0f;
    float codes[QWREF_GROUP];
    for (uint32_t g = 0; g < cols / QWREF_GROUP; ++g) {
        float scale = qwref_from_f16(read_f16_le(row_scales, g));
        dequantize_group(format, row_data + (size_t)g * data_bytes, scale, codes);
        const float *activations = x + (size_t)g * QWREF_GROUP;
        for (int i = 0; i < QWREF_GROUP; ++i) accumulator += codes[i] * activations[i];
    }
    return accumulator;
}

uint64_t qwref_fnv1a64(const uint8_t *bytes, uint64_t len, uint64_t state) {
    for (uint64_t i = 0; i < len; ++i) {
        state ^= bytes[i];
        state *= 0x100000001b3ull;
    }
    return state;
}

/* selftest.zig:73-126 `checkQuantization`: the golden pattern
 * f32(cos(f32(i) * 0.19)) * 1.75 packed as q4, q5, q8, FNV-1a over each
 * format's scale plane then code plane. Zig's @cos is its compiler_rt cosf;
 * glibc cosf is used here (the golden hash pins whether they agree). */
uint64_t qwref_quant_hash(void) {
    enum { cols = 128 };
    float values[cols];
    for (int i = 0; i < cols; ++i) {
        float position = (float)i;
        values[i] = cosf(position * 0.19f) * 1.75f;
    }
    uint64_t hash = 0xcbf29ce484222325ull;
    const int32_t formats[3] = {QWREF_Q4, QWREF_Q5, QWREF_Q8};
    for (int f = 0; f < 3; ++f) {
        uint8_t scales[cols / QWREF_GROUP * 2];
        uint8_t data[cols / QWREF_GROUP * 64];
        size_t data_len = (size_t)(cols / QWREF_GROUP) * (size_t)qwref_data_bytes_per_group(formats[f]);
        qwref_quantize_row(formats[f], values, cols, scales, data);
        hash = qwref_fnv1a64(scales, sizeof scales, hash);
        hash = qwref_fnv1a64(data, data_len, hash);
    }
    return hash;
}

/* ------------------------------------------------------------------------ */
/* kernels.zig                                                               */
/* ------------------------------------------------------------------------ */

/* kernels.zig:39-51 `dotF32`: four f32 lanes, lane j sums elements j, j+4,
 * ...; then @reduce(.Add) taken in lane order; then a scalar tail. */
float qwref_dot_f32(const float *left, const float *right, uint32_t len) {
    float acc0 = 0.0f, acc1 = 0.0f, acc2 = 0.0f, acc3 = 0.0f;
    uint32_t index = 0;
    for (; index + 4 <= len; index += 4) {
        acc0 += left[index + 0] * right[index + 0];
        acc1 += left[index + 1] * right[index + 1];
        acc2 += left[index + 2] * right[index + 2];
        acc3 += left[index + 3] * right[index + 3];
    }
    float total = ((acc0 + acc1) + acc2) + acc3;
    for (; index < len; ++index) total += left[index] * right[index];
    return total;
}

/* kernels.zig:54-75 `linearF32`. */
int32_t qwref_linear_f32(float *out, const float *x, const float *weights, uint32_t rows,
                         uint32_t cols, uint32_t tokens) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t row = 0; row < (int64_t)rows; ++row)
        for (uint32_t token = 0; token < tokens; ++token)
            out[(size_t)token * rows + row] =
                qwref_dot_f32(weights + (size_t)row * cols, x + (size_t)token * cols, cols);
    return QWREF_OK;
}

/* kernels.zig:82-112 `linearF16`: each weight row widened into scratch
 * (half_float.fromF16), then dotF32 against every token. Rows are
 * independent, so the optional thread split changes no output's
 * arithmetic. */
int32_t qwref_linear_f16(float *out, const float *x, const uint16_t *weights, uint32_t rows,
                         uint32_t cols, uint32_t tokens) {
    int32_t status = QWREF_OK;
#pragma omp parallel num_threads(g_threads)
    {
        float *scratch = (float *)malloc(sizeof(float) * (cols ? cols : 1));
        if (!scratch) {
#pragma omp atomic write
            status = QWREF_LIMIT_EXCEEDED;
        }
#pragma omp for schedule(static)
        for (int64_t row = 0; row < (int64_t)rows; ++row) {
            if (!scratch) continue;
            for (uint32_t k = 0; k < cols; ++k) scratch[k] = qwref_from_f16(weights[(size_t)row * cols + k]);
            for (uint32_t token = 0; token < tokens; ++token)
                out[(size_t)token * rows + row] = qwref_dot_f32(scratch, x + (size_t)token * cols, cols);
        }
        free(scratch);
    }
    return status;
}

/* kernels.zig:118-158 `linearQuantized` (reached through Matrix.apply,
 * kernels.zig:182-206): shape checks, then per row dequantizeRow into
 * scratch and dotF32 against every token. Rows are independent, so the
 * optional thread split changes nothing about any output's arithmetic. */
int32_t qwref_linear_quantized(float *out, const float *x, int32_t format, const uint8_t *scales,
                               uint64_t scales_len, const uint8_t *data, uint64_t data_len,
                               uint32_t rows, uint32_t cols, uint32_t tokens) {
    if (cols % QWREF_GROUP != 0) return QWREF_SHAPE_MISMATCH;
    uint32_t gpr = cols / QWREF_GROUP;
    int32_t data_bytes = qwref_data_bytes_per_group(format);
    if (data_bytes == 0) return QWREF_UNSUPPORTED;
    if (scales_len != (uint64_t)rows * gpr * 2u) return QWREF_SHAPE_MISMATCH;
    if (data_len != (uint64_t)rows * gpr * (uint64_t)data_bytes) return QWREF_SHAPE_MISMATCH;
#pragma omp parallel num_threads(g_threads)
    {
        float *scratch = (float *)malloc(sizeof(float) * cols);
#pragma omp for schedule(static)
        for (int64_t row = 0; row < (int64_t)rows; ++row) {
            qwref_dequantize_row(format, scales + (size_t)row * gpr * 2,
                                 data + (size_t)row * gpr * (size_t)data_bytes, scratch, cols);
            for (uint32_t token = 0; token < tokens; ++token)
                out[(size_t)token * rows + (size_t)row] =
                    qwref_dot_f32(scratch, x + (size_t)token * cols, cols);
        }
        free(scratch);
    }
    return QWREF_OK;
}

/* kernels.zig:221-230 `addInPlace`. */
void qwref_add_in_place(float *x, const float *y, uint32_t len) {
    for (uint32_t i = 0; i < len; ++i) x[i] += y[i];
}

/* math.zig:69-71 `silu`. */
float qwref_silu(float x) { return x / (1.0f + expf(-x)); }

/* kernels.zig:233-239 `siluMul`. */
void qwref_silu_mul(float *out, const float *gate, const float *up, uint32_t len) {
    for (uint32_t i = 0; i < len; ++i) out[i] = qwref_silu(gate[i]) * up[i];
}

/* math.zig:77-93 `softmaxInPlace`. */
void qwref_softmax_in_place(float *row, uint32_t len) {
    float row_max = row[0];
    for (uint32_t i = 1; i < len; ++i) row_max = row[i] > row_max ? row[i] : row_max;
    float total = 0.0f;
    for (uint32_t i = 0; i < len; ++i) {
        row[i] = expf(row[i] - row_max);
        total += row[i];
    }
    float inverse_total = 1.0f / total;
    for (uint32_t i = 0; i < len; ++i) row[i] *= inverse_total;
}

/* math.zig:120-130 `rmsNormInPlace`, via kernels.zig:288-300 `rmsNorm`. */
void qwref_rms_norm(float *x, const float *weight, uint32_t width, uint32_t tokens, float eps) {
    for (uint32_t t = 0; t < tokens; ++t) {
        float *row = x + (size_t)t * width;
        float sum_squares = 0.0f;
        for (uint32_t i = 0; i < width; ++i) sum_squares += row[i] * row[i];
        float mean_square = sum_squares / (float)width;
        float inverse_rms = 1.0f / sqrtf(mean_square + eps);
        for (uint32_t i = 0; i < width; ++i) row[i] = row[i] * inverse_rms * weight[i];
    }
}

/* kernels.zig:561-564 `inverseFrequency`: theta ^ (-2i / head_dim) in f32.
 * std.math.pow(f32) is restated by powf (last-ulp parity unpinned). */
float qwref_inverse_frequency(uint32_t index, uint32_t head_dim, float theta) {
    float exponent = -2.0f * (float)index / (float)head_dim;
    return powf(theta, exponent);
}

/* kernels.zig:534-558 `buildRopeTables`. */
void qwref_build_rope_tables(float *cos_table, float *sin_table, uint32_t half, float theta,
                             uint32_t max_positions, uint32_t stride) {
    uint32_t head_dim = half * 2;
    for (uint32_t position = 0; position < max_positions; ++position) {
        for (uint32_t index = 0; index < half; ++index) {
            float angle = (float)position * qwref_inverse_frequency(index, head_dim, theta);
            size_t offset = (size_t)position * stride + index;
            cos_table[offset] = cosf(angle);
            sin_table[offset] = sinf(angle);
        }
    }
}

/* kernels.zig:495-527 `ropeInPlace`: rotate_half pairing (i, i + half). */
void qwref_rope_in_place(float *rotated, const uint32_t *positions, uint32_t tokens,
                         uint32_t heads, uint32_t head_dim, const float *cos_table,
                         const float *sin_table, uint32_t table_stride) {
    uint32_t width = heads * head_dim;
    uint32_t half = head_dim / 2;
    for (uint32_t token = 0; token < tokens; ++token) {
        const float *cos_row = cos_table + (size_t)positions[token] * table_stride;
        const float *sin_row = sin_table + (size_t)positions[token] * table_stride;
        for (uint32_t head = 0; head < heads; ++head) {
            float *row = rotated + (size_t)token * width + (size_t)head * head_dim;
            for (uint32_t i = 0; i < half; ++i) {
                float low = row[i];
                float high = row[i + half];
                row[i] = low * cos_row[i] - high * sin_row[i];
                row[i + half] = high * cos_row[i] + low * sin_row[i];
            }
        }
    }
}

/* kernels.zig:572-627 `decodeAttentionStep` (f32 cache). */
int32_t qwref_decode_attention_step(float *out, const float *query, const float *keys,
                                    const float *values, uint32_t cached, uint32_t heads,
                                    uint32_t kv_heads, uint32_t head_dim) {
    if (kv_heads == 0 || heads % kv_heads != 0) return QWREF_SHAPE_MISMATCH;
    if (cached == 0) return QWREF_SHAPE_MISMATCH;
    uint32_t kv_width = kv_heads * head_dim;
    uint32_t groups = heads / kv_heads;
    float scaling = 1.0f / sqrtf((float)head_dim);
    float *scores = (float *)malloc(sizeof(float) * cached);
    for (uint32_t head = 0; head < heads; ++head) {
        const float *hq = query + (size_t)head * head_dim;
        uint32_t kvh = head / groups;
        for (uint32_t p = 0; p < cached; ++p)
            scores[p] = qwref_dot_f32(hq, keys + (size_t)p * kv_width + (size_t)kvh * head_dim, head_dim) * scaling;
        qwref_softmax_in_place(scores, cached);
        float *ho = out + (size_t)head * head_dim;
        memset(ho, 0, sizeof(float) * head_dim);
        for (uint32_t p = 0; p < cached; ++p) {
            const float *vr = values + (size_t)p * kv_width + (size_t)kvh * head_dim;
            float w = scores[p];
            for (uint32_t i = 0; i < head_dim; ++i) ho[i] = ho[i] + vr[i] * w;
        }
    }
    free(scores);
    return QWREF_OK;
}

/* kernels.zig:636-661 `q8GroupDot`: per group a four-lane inner sum of
 * (u - 128) * q, reduced in lane order, times the group's scale, added to a
 * running f32 total. */
static float q8_group_dot(const float *query_row, const uint8_t *codes, const uint8_t *scales,
                          size_t first_group, uint32_t groups) {
    float total = 0.0f;
    for (uint32_t g = 0; g < groups; ++g) {
        size_t base = (size_t)g * QWREF_GROUP;
        float scale = qwref_from_f16(read_f16_le(scales, first_group + g));
        float in0 = 0.0f, in1 = 0.0f, in2 = 0.0f, in3 = 0.0f;
        for (int i = 0; i < QWREF_GROUP; i += 4) {
            in0 += ((float)codes[base + i + 0] - 128.0f) * query_row[base + i + 0];
            in1 += ((float)codes[base + i + 1] - 128.0f) * query_row[base + i + 1];
            in2 += ((float)codes[base + i + 2] - 128.0f) * query_row[base + i + 2];
            in3 += ((float)codes[base + i + 3] - 128.0f) * query_row[base + i + 3];
        }
        total += (((in0 + in1) + in2) + in3) * scale;
    }
    return total;
}

/* kernels.zig:665-688 `q8GroupAccumulate`: out += (u - 128) * (scale * weight). */
static void q8_group_accumulate(float *out_row, const uint8_t *codes, const uint8_t *scales,
                                size_t first_group, uint32_t groups, float weight) {
    for (uint32_t g = 0; g < groups; ++g) {
        size_t base = (size_t)g * QWREF_GROUP;
        float scale = qwref_from_f16(read_f16_le(scales, first_group + g));
        float scaled_weight = scale * weight;
        for (int i = 0; i < QWREF_GROUP; ++i)
            out_row[base + i] = out_row[base + i] + ((float)codes[base + i] - 128.0f) * scaled_weight;
    }
}

/* kernels.zig:697-767 `decodeAttentionStepQ8`. */
int32_t qwref_decode_attention_step_q8(float *out, const float *query, const uint8_t *k_scales,
                                       const uint8_t *k_codes, const uint8_t *v_scales,
                                       const uint8_t *v_codes, uint32_t cached, uint32_t heads,
                                       uint32_t kv_heads, uint32_t head_dim) {
    if (head_dim % QWREF_GROUP != 0) return QWREF_SHAPE_MISMATCH;
    if (kv_heads == 0 || heads % kv_heads != 0) return QWREF_SHAPE_MISMATCH;
    if (cached == 0) return QWREF_SHAPE_MISMATCH;
    uint32_t kv_width = kv_heads * head_dim;
    uint32_t groups_per_row = kv_width / QWREF_GROUP;
    uint32_t groups = heads / kv_heads;
    uint32_t groups_per_head = head_dim / QWREF_GROUP;
    float scaling = 1.0f / sqrtf((float)head_dim);
#pragma omp parallel num_threads(g_threads)
    {
        float *scores = (float *)malloc(sizeof(float) * cached);
#pragma omp for schedule(static)
        for (int64_t head = 0; head < (int64_t)heads; ++head) {
            const float *hq = query + (size_t)head * head_dim;
            uint32_t kvh = (uint32_t)head / groups;
            size_t head_group = (size_t)kvh * head_dim / QWREF_GROUP;
            for (uint32_t p = 0; p < cached; ++p) {
                size_t row_group = (size_t)p * groups_per_row + head_group;
                const uint8_t *codes = k_codes + (size_t)p * kv_width + (size_t)kvh * head_dim;
                scores[p] = scaling * q8_group_dot(hq, codes, k_scales, row_group, groups_per_head);
            }
            qwref_softmax_in_place(scores, cached);
            float *ho = out + (size_t)head * head_dim;
            memset(ho, 0, sizeof(float) * head_dim);
            for (uint32_t p = 0; p < cached; ++p) {
                size_t row_group = (size_t)p * groups_per_row + head_group;
                const uint8_t *codes = v_codes + (size_t)p * kv_width + (size_t)kvh * head_dim;
                q8_group_accumulate(ho, codes, v_scales, row_group, groups_per_head, scores[p]);
            }
        }
        free(scores);
    }
    return QWREF_OK;
}

/* decoder.zig:290-301 `argmaxLogits`: the first maximum wins (strict >). */
uint32_t qwref_argmax(const float *logits, uint32_t count) {
    uint32_t best = 0;
    float best_value = logits[0];
    for (uint32_t i = 1; i < count; ++i) {
        if (logits[i] > best_value) {
            best_value = logits[i];
            best = i;
        }
    }
    return best;
}

/* ------------------------------------------------------------------------ */
/* Audio tower glue                                                          */
/* ------------------------------------------------------------------------ */

/* math.zig:46-60 `erf`: the Chebyshev fit of erfc from Numerical Recipes
 * (`erfcc`, fractional error below 1.2e-7), in f32, with expf standing in for
 * the reference's exp (last-ulp parity unpinned). */
float qwref_erf(float x) {
    float sign = x < 0.0f ? -1.0f : 1.0f;
    float magnitude = fabsf(x);
    float t = 1.0f / (1.0f + 0.5f * magnitude);
    float poly = -0.82215223f + t * 0.17087277f;
    poly = 1.48851587f + t * poly;
    poly = -1.13520398f + t * poly;
    poly = 0.27886807f + t * poly;
    poly = -0.18628806f + t * poly;
    poly = 0.09678418f + t * poly;
    poly = 0.37409196f + t * poly;
    poly = 1.00002368f + t * poly;
    float tau = t * expf(-magnitude * magnitude - 1.26551223f + t * poly);
    return sign * (1.0f - tau);
}

/* math.zig:63-66 `gelu` (exact, error-function form). */
float qwref_gelu(float x) {
    const float inverse_sqrt_two = 0.70710678f;
    return 0.5f * x * (1.0f + qwref_erf(x * inverse_sqrt_two));
}

/* model.zig:719 / :868: GELU applied over a whole projection output. */
void qwref_gelu_in_place(float *x, uint64_t len) {
    for (uint64_t i = 0; i < len; ++i) x[i] = qwref_gelu(x[i]);
}

/* kernels.zig:210-218 `addBias`: x[t][r] += bias[r]. */
int32_t qwref_add_bias(float *x, const float *bias, uint32_t rows, uint32_t tokens) {
    for (uint32_t t = 0; t < tokens; ++t) {
        float *row = x + (size_t)t * rows;
        for (uint32_t r = 0; r < rows; ++r) row[r] += bias[r];
    }
    return 0;
}

/* math.zig:99-116 `layerNormInPlace`, per token as kernels.zig:242-255
 * `layerNorm`: mean, centred variance, 1/sqrt(variance + eps), then
 * (x - mean) * inverse_std * weight + bias, each in f32 and in that order. */
void qwref_layer_norm(float *x, const float *weight, const float *bias, uint32_t width, uint32_t tokens,
                      float eps) {
    for (uint32_t t = 0; t < tokens; ++t) {
        float *row = x + (size_t)t * width;
        float sum = 0.0f;
        for (uint32_t i = 0; i < width; ++i) sum += row[i];
        float mean = sum / (float)width;
        float sum_squares = 0.0f;
        for (uint32_t i = 0; i < width; ++i) {
            float centered = row[i] - mean;
            sum_squares += centered * centered;
        }
        float variance = sum_squares / (float)width;
        float inverse_std = 1.0f / sqrtf(variance + eps);
        for (uint32_t i = 0; i < width; ++i) row[i] = (row[i] - mean) * inverse_std * weight[i] + bias[i];
    }
}

/* kernels.zig:429-484 `audioAttentionWindow`: non-causal attention of every
 * query in [window_start, window_start + window_length) over the keys of the
 * same range, per head; rows `stride` floats apart. Scores are dotF32 times
 * 1/sqrt(head_dim), softmaxInPlace, then out_row = sum_k weight_k * v_k with
 * the reference's 4-lane vector accumulate (lane-wise, so element order). */
int32_t qwref_audio_attention_window(float *out, uint32_t out_stride, const float *q, uint32_t q_stride,
                                     const float *k, uint32_t k_stride, const float *v, uint32_t v_stride,
                                     uint32_t window_start, uint32_t window_length, uint32_t heads,
                                     uint32_t head_dim) {
    if (window_length == 0) return -7;
    float *scores = (float *)malloc(sizeof(float) * window_length);
    if (!scores) return -2;
    const float scaling = 1.0f / sqrtf((float)head_dim);
    for (uint32_t head = 0; head < heads; ++head) {
        for (uint32_t query = 0; query < window_length; ++query) {
            const float *query_row = q + (size_t)(window_start + query) * q_stride + (size_t)head * head_dim;
            for (uint32_t key = 0; key < window_length; ++key) {
                const float *key_row = k + (size_t)(window_start + key) * k_stride + (size_t)head * head_dim;
                scores[key] = qwref_dot_f32(query_row, key_row, head_dim) * scaling;
            }
            qwref_softmax_in_place(scores, window_length);
            float *out_row = out + (size_t)(window_start + query) * out_stride + (size_t)head * head_dim;
            for (uint32_t i = 0; i < head_dim; ++i) out_row[i] = 0.0f;
            for (uint32_t key = 0; key < window_length; ++key) {
                const float *value_row = v + (size_t)(window_start + key) * v_stride + (size_t)head * head_dim;
                const float weight = scores[key];
                for (uint32_t i = 0; i < head_dim; ++i) out_row[i] = out_row[i] + value_row[i] * weight;
            }
        }
    }
    free(scores);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Synthetic inputs. Not reference code: the seeded-input specification the  */
/* oracle and the HIP backend both implement (independently) so that large    */
/* configurations can be generated on either side and compared bit for bit.  */
/*                                                                            */
/*   draw n (n >= 1) of a stream with base b: mulberry32 output of state      */
/*     b + n * 0x6d2b79f5 (the generator of tests/gpu/reference.mjs:35-44,   */
/*     which is counter based: state n is b + n * increment).                 */
/*   stream base: seed + stream * 0x9e3779b9 (mod 2^32).                      */
/*   normal value i: draws 2i+1 and 2i+2, Box-Muller as reference.mjs:54-58:  */
/*     f32( sqrt(-2 ln(1 - u1/2^32)) * cos(2 pi u2/2^32) )                    */
/*   with ln, cos and sqrt evaluated in double by the fixed operation         */
/*   sequences below (IEEE + - * / only, no fused operations), so that the    */
/*   CPU and the GPU compute identical bits.                                  */
/* ------------------------------------------------------------------------ */

static uint32_t mulberry32_output(uint32_t state) {
    uint32_t value = state;
    value = (value ^ (value >> 15)) * (value | 1u);
    value = value ^ (value + (value ^ (value >> 7)) * (value | 61u));
    return value ^ (value >> 14);
}

uint32_t qwref_stream_base(uint32_t seed, uint32_t stream) { return seed + stream * 0x9e3779b9u; }

uint32_t qwref_mulberry32_at(uint32_t base, uint64_t draw) {
    return mulberry32_output(base + (uint32_t)draw * 0x6d2b79f5u);
}

static uint64_t f64_bits(double v) {
    uint64_t b;
    memcpy(&b, &v, 8);
    return b;
}

static double bits_f64(uint64_t b) {
    double v;
    memcpy(&v, &b, 8);
    return v;
}

/* ln x for x in (0, 1]: x = m 2^e with m in (sqrt(1/2), sqrt(2)],
 * ln m = 2 atanh(s), s = (m-1)/(m+1), series to s^23. */
static double det_log(double x) {
    uint64_t bits = f64_bits(x);
    int32_t e = (int32_t)((bits >> 52) & 0x7ff) - 1023;
    double m = bits_f64((bits & 0x000fffffffffffffull) | 0x3ff0000000000000ull);
    if (m > 1.4142135623730951) {
        m = m * 0.5;
        e = e + 1;
    }
    double s = (m - 1.0) / (m + 1.0);
    double z = s * s;
    double p = 1.0 / 23.0;
    p = p * z + 1.0 / 21.0;
    p = p * z + 1.0 / 19.0;
    p = p * z + 1.0 / 17.0;
    p = p * z + 1.0 / 15.0;
    p = p * z + 1.0 / 13.0;
    p = p * z + 1.0 / 11.0;
    p = p * z + 1.0 / 9.0;
    p = p * z + 1.0 / 7.0;
    p = p * z + 1.0 / 5.0;
    p = p * z + 1.0 / 3.0;
    p = p * z + 1.0;
    double log_m = (2.0 * s) * p;
    double de = (double)e;
    return de * 6.93147180369123816490e-01 + (de * 1.90821492927058770002e-10 + log_m);
}

/* cos(2 pi t) for t in [0, 1): exact quadrant split of 4t, reduction to an
 * angle in [0, pi/4], Taylor series to degree 20/21. */
static double det_cos2pi(double t) {
    double q4 = t * 4.0;
    int32_t q = (int32_t)q4;
    double f = q4 - (double)q;
    int32_t use_sin = q & 1;
    double g = f;
    if (f > 0.5) {
        g = 1.0 - f;
        use_sin = !use_sin;
    }
    double y = g * 1.5707963267948966;
    double y2 = y * y;
    double r;
    if (use_sin) {
        double p = 1.0 / 51090942171709440000.0;
        p = p * y2 - 1.0 / 121645100408832000.0;
        p = p * y2 + 1.0 / 355687428096000.0;
        p = p * y2 - 1.0 / 1307674368000.0;
        p = p * y2 + 1.0 / 6227020800.0;
        p = p * y2 - 1.0 / 39916800.0;
        p = p * y2 + 1.0 / 362880.0;
        p = p * y2 - 1.0 / 5040.0;
        p = p * y2 + 1.0 / 120.0;
        p = p * y2 - 1.0 / 6.0;
        p = p * y2 + 1.0;
        r = y * p;
    } else {
        double p = 1.0 / 2432902008176640000.0;
        p = p * y2 - 1.0 / 6402373705728000.0;
        p = p * y2 + 1.0 / 20922789888000.0;
        p = p * y2 - 1.0 / 87178291200.0;
        p = p * y2 + 1.0 / 479001600.0;
        p = p * y2 - 1.0 / 3628800.0;
        p = p * y2 + 1.0 / 40320.0;
        p = p * y2 - 1.0 / 720.0;
        p = p * y2 + 1.0 / 24.0;
        p = p * y2 - 1.0 / 2.0;
        p = p * y2 + 1.0;
        r = p;
    }
    return (q == 1 || q == 2) ? -r : r;
}

/* sqrt y, y >= 0: exponent-halving first guess, six Newton steps. */
static double det_sqrt(double y) {
    if (y == 0.0) return 0.0;
    double g = bits_f64((f64_bits(y) >> 1) + 0x1ff8000000000000ull);
    for (int i = 0; i < 6; ++i) g = 0.5 * (g + y / g);
    return g;
}

float qwref_normal_at(uint32_t seed, uint32_t stream, uint64_t index) {
    uint32_t base = qwref_stream_base(seed, stream);
    uint32_t u1 = qwref_mulberry32_at(base, 2 * index + 1);
    uint32_t u2 = qwref_mulberry32_at(base, 2 * index + 2);
    double first = 1.0 - (double)u1 / 4294967296.0;
    double second = (double)u2 / 4294967296.0;
    double radius = det_sqrt(-2.0 * det_log(first));
    return (float)(radius * det_cos2pi(second));
}

void qwref_fill_normal(float *out, uint64_t count, uint32_t seed, uint32_t stream, float scale) {
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int64_t i = 0; i < (int64_t)count; ++i) out[i] = qwref_normal_at(seed, stream, (uint64_t)i) * scale;
}

/* ------------------------------------------------------------------------ */
/* Audio convolution front end (kernels.zig:302-427, model.zig:509-644,     */
/* :751-763; model_config.zig:84-90)                                         */
/* ------------------------------------------------------------------------ */

/* model_config.zig:84-90 `postConvolutionSteps`: three (n - 1) / 2 + 1. */
uint32_t qwref_post_convolution_steps(uint32_t frames) {
    if (frames == 0) return 0;
    uint32_t steps = frames;
    for (int i = 0; i < 3; ++i) steps = (steps - 1) / 2 + 1;
    return steps;
}

/* kernels.zig:386-427 `convolvePlane`: adds one input channel's 3x3 stride-2
 * padding-1 contribution to an output plane; per output position the nine
 * taps are summed in kernel order (taps outside the input skipped), then the
 * sum is added to the output. */
static void convolve_plane(float *out, const float *input, const uint16_t *weights, uint32_t in_height,
                           uint32_t in_width) {
    uint32_t out_height = (in_height - 1) / 2 + 1, out_width = (in_width - 1) / 2 + 1;
    float kernel_weights[9];
    for (int i = 0; i < 9; ++i) kernel_weights[i] = qwref_from_f16(weights[i]);
    for (uint32_t out_row = 0; out_row < out_height; ++out_row) {
        for (uint32_t out_column = 0; out_column < out_width; ++out_column) {
            float accumulator = 0.0f;
            for (int kernel_row = 0; kernel_row < 3; ++kernel_row) {
                int64_t in_row = (int64_t)out_row * 2 + kernel_row - 1;
                if (in_row < 0 || in_row >= (int64_t)in_height) continue;
                for (int kernel_column = 0; kernel_column < 3; ++kernel_column) {
                    int64_t in_column = (int64_t)out_column * 2 + kernel_column - 1;
                    if (in_column < 0 || in_column >= (int64_t)in_width) continue;
                    float sample = input[(size_t)in_row * in_width + (size_t)in_column];
                    accumulator += kernel_weights[kernel_row * 3 + kernel_column] * sample;
                }
            }
            out[(size_t)out_row * out_width + out_column] += accumulator;
        }
    }
}

/* kernels.zig:325-384 `conv3x3Stride2Gelu` / `convolveChannel`: per output
 * channel the plane starts at the bias, every input channel's contribution is
 * added in channel order, then GELU. Weights [out][in][3][3] f16 bits, input
 * [in][h][w], output [out][oh][ow]. */
int32_t qwref_conv3x3s2_gelu(float *out, const float *input, const uint16_t *weights, const float *bias,
                             uint32_t out_channels, uint32_t in_channels, uint32_t in_height, uint32_t in_width) {
    if (in_height == 0 || in_width == 0 || in_channels == 0) return QWREF_SHAPE_MISMATCH;
    uint32_t out_height = (in_height - 1) / 2 + 1, out_width = (in_width - 1) / 2 + 1;
    size_t in_plane = (size_t)in_height * in_width, out_plane = (size_t)out_height * out_width;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int64_t channel = 0; channel < (int64_t)out_channels; ++channel) {
        float *out_slice = out + (size_t)channel * out_plane;
        for (size_t i = 0; i < out_plane; ++i) out_slice[i] = bias[channel];
        const uint16_t *weight_base = weights + (size_t)channel * in_channels * 9;
        for (uint32_t in_channel = 0; in_channel < in_channels; ++in_channel)
            convolve_plane(out_slice, input + (size_t)in_channel * in_plane, weight_base + (size_t)in_channel * 9,
                           in_height, in_width);
        for (size_t i = 0; i < out_plane; ++i) out_slice[i] = qwref_gelu(out_slice[i]);
    }
    return QWREF_OK;
}

/* model.zig:751-763 `addSinusoidalPosition`: inverse timescales and angles in
 * f64, each sine / cosine narrowed to f32 and added to the row. */
void qwref_add_sinusoidal_position(float *row, uint32_t step, uint32_t channels) {
    uint32_t half = channels / 2;
    double log_timescale_increment = log(10000.0) / ((double)half - 1.0);
    double position = (double)step;
    for (uint32_t index = 0; index < half; ++index) {
        double inverse_timescale = exp(-log_timescale_increment * (double)index);
        double angle = position * inverse_timescale;
        row[index] += (float)sin(angle);
        row[half + index] += (float)cos(angle);
    }
}

/* ------------------------------------------------------------------------ */
/* decoder.zig restatement with a synthetic q4 model and q8 cache            */
/* ------------------------------------------------------------------------ */

typedef struct {
    int32_t format; /* QWREF_Q4, QWREF_Q5, QWREF_Q8, or QWREF_F32 / QWREF_F16
                       (kernels.zig:161-166: the elements in `data`, no scales) */
    uint8_t *scales;
    uint8_t *data;
    uint64_t scales_len;
    uint64_t data_len;
    uint32_t rows;
    uint32_t cols;
} qmat;

typedef struct {
    qmat q, k, v, o, gate, up, down;
    /* decoder.zig:165-172, :180-193, :259-265: the layer's four norm weights */
    float *attention_norm, *q_norm, *k_norm, *ffn_norm;
} layer_mats;

typedef struct {
    /* q8: layers x [max_pos x groups x 2 B scales][max_pos x kv_width codes]
     * (decoder.zig:58-65); f32: layers x [max_pos x kv_width] f32
     * (decoder.zig:77-83). */
    uint8_t *keys;
    uint8_t *values;
    uint32_t position;
    float *logits;
} sequence_state;

struct qwref_decoder {
    qwref_decoder_config c;
    uint32_t seed;
    uint32_t batch;
    int32_t weight_format;
    int32_t cache_format; /* QWREF_CACHE_F32 or QWREF_CACHE_Q8 (model_config.zig:44-68) */
    qmat embed, lm_head;
    layer_mats *layers;
    float *final_norm;
    float *rope_cos, *rope_sin;
    sequence_state *seqs;
    /* scratch, as model.zig:1063-1072 */
    float *hidden, *normed, *query, *key, *value, *attention_out, *gate, *up;
    size_t cache_scales, cache_codes, cache_stride;
};

/* Stream ids of the synthetic model (seed given by the caller). */
enum {
    STREAM_EMBED = 1,
    STREAM_LM_HEAD = 2,
    STREAM_LAYER_BASE = 16, /* + 16 * layer + {0 q,1 k,2 v,3 o,4 gate,5 up,6 down} */
    STREAM_CACHE_BASE = 0x10000, /* + 0x100 * seq + 2 * layer + {0 keys, 1 values} */
    STREAM_START_TOKEN = 0x20000, /* + seq */
};

static int make_qmat(qmat *m, int32_t format, uint32_t rows, uint32_t cols, uint32_t seed, uint32_t stream) {
    m->format = format;
    m->rows = rows;
    m->cols = cols;
    if (format == QWREF_F32 || format == QWREF_F16) {
        /* The generator's values as they are, or rounded to f16
         * (half_float.zig:14-17). */
        const uint64_t count = (uint64_t)rows * cols;
        m->scales = NULL;
        m->scales_len = 0;
        m->data_len = count * (format == QWREF_F32 ? 4u : 2u);
        m->data = (uint8_t *)malloc(m->data_len);
        if (!m->data) return -1;
        if (format == QWREF_F32) {
            qwref_fill_normal((float *)m->data, count, seed, stream, 0.02f);
            return 0;
        }
        float *values = (float *)malloc(sizeof(float) * count);
        if (!values) return -1;
        qwref_fill_normal(values, count, seed, stream, 0.02f);
        uint16_t *bits = (uint16_t *)m->data;
        for (uint64_t i = 0; i < count; ++i) bits[i] = qwref_to_f16(values[i]);
        free(values);
        return 0;
    }
    m->scales_len = (uint64_t)rows * (cols / QWREF_GROUP) * 2u;
    m->data_len = (uint64_t)rows * (cols / QWREF_GROUP) * (uint64_t)qwref_data_bytes_per_group(format);
    m->scales = (uint8_t *)malloc(m->scales_len);
    m->data = (uint8_t *)malloc(m->data_len);
    float *values = (float *)malloc(sizeof(float) * (size_t)rows * cols);
    if (!m->scales || !m->data || !values) {
        free(values);
        return -1;
    }
    qwref_fill_normal(values, (uint64_t)rows * cols, seed, stream, 0.02f);
    qwref_quantize_rows(format, values, rows, cols, m->scales, m->data);
    free(values);
    return 0;
}

static void free_qmat(qmat *m) {
    free(m->scales);
    free(m->data);
}

static float *ones(uint32_t count) {
    float *v = (float *)malloc(sizeof(float) * count);
    for (uint32_t i = 0; i < count; ++i) v[i] = 1.0f;
    return v;
}

uint32_t qwref_synthetic_start_token(uint32_t seed, uint32_t seq, uint32_t vocab) {
    return qwref_mulberry32_at(qwref_stream_base(seed, STREAM_START_TOKEN + seq), 1) % vocab;
}

qwref_decoder *qwref_decoder_create_synthetic(const qwref_decoder_config *config, uint32_t seed,
                                              uint32_t batch) {
    return qwref_decoder_create_synthetic_as(config, seed, batch, QWREF_Q4, QWREF_CACHE_Q8);
}

qwref_decoder *qwref_decoder_create_synthetic_as(const qwref_decoder_config *config, uint32_t seed,
                                                 uint32_t batch, int32_t weight_format,
                                                 int32_t cache_format) {
    if (qwref_data_bytes_per_group(weight_format) == 0 && weight_format != QWREF_F32 && weight_format != QWREF_F16)
        return NULL;
    if (cache_format != QWREF_CACHE_F32 && cache_format != QWREF_CACHE_Q8) return NULL;
    qwref_decoder *d = (qwref_decoder *)calloc(1, sizeof *d);
    d->c = *config;
    d->seed = seed;
    d->batch = batch;
    d->weight_format = weight_format;
    d->cache_format = cache_format;
    const qwref_decoder_config *c = config;
    int32_t f = weight_format;
    uint32_t qw = c->heads * c->head_dim, kvw = c->kv_heads * c->head_dim;
    make_qmat(&d->embed, f, c->vocab, c->hidden, seed, STREAM_EMBED);
    make_qmat(&d->lm_head, f, c->vocab, c->hidden, seed, STREAM_LM_HEAD);
    d->layers = (layer_mats *)calloc(c->layers, sizeof(layer_mats));
    for (uint32_t l = 0; l < c->layers; ++l) {
        uint32_t s = STREAM_LAYER_BASE + 16 * l;
        layer_mats *m = &d->layers[l];
        make_qmat(&m->q, f, qw, c->hidden, seed, s + 0);
        make_qmat(&m->k, f, kvw, c->hidden, seed, s + 1);
        make_qmat(&m->v, f, kvw, c->hidden, seed, s + 2);
        make_qmat(&m->o, f, c->hidden, qw, seed, s + 3);
        make_qmat(&m->gate, f, c->ffn, c->hidden, seed, s + 4);
        make_qmat(&m->up, f, c->ffn, c->hidden, seed, s + 5);
        make_qmat(&m->down, f, c->hidden, c->ffn, seed, s + 6);
        /* Norm weights start at 1.0; qwref_decoder_set_vector replaces them. */
        m->attention_norm = ones(c->hidden);
        m->ffn_norm = ones(c->hidden);
        m->q_norm = ones(c->head_dim);
        m->k_norm = ones(c->head_dim);
    }
    d->final_norm = ones(c->hidden);
    uint32_t half = c->head_dim / 2;
    d->rope_cos = (float *)malloc(sizeof(float) * (size_t)c->max_positions * half);
    d->rope_sin = (float *)malloc(sizeof(float) * (size_t)c->max_positions * half);
    /* model.zig:400-407 */
    qwref_build_rope_tables(d->rope_cos, d->rope_sin, half, c->theta, c->max_positions, half);
    if (cache_format == QWREF_CACHE_Q8) {
        /* decoder.zig:58-65 `cachePlane` */
        d->cache_scales = (size_t)c->max_positions * (kvw / QWREF_GROUP) * 2u;
        d->cache_codes = (size_t)c->max_positions * kvw;
    } else {
        /* decoder.zig:77-83: one f32 per element, layer stride max_pos * kv_width */
        d->cache_scales = 0;
        d->cache_codes = (size_t)c->max_positions * kvw * sizeof(float);
    }
    d->cache_stride = d->cache_scales + d->cache_codes;
    d->seqs = (sequence_state *)calloc(batch, sizeof(sequence_state));
    for (uint32_t b = 0; b < batch; ++b) {
        d->seqs[b].keys = (uint8_t *)calloc((size_t)c->layers, d->cache_stride);
        d->seqs[b].values = (uint8_t *)calloc((size_t)c->layers, d->cache_stride);
        d->seqs[b].logits = (float *)calloc(c->vocab, sizeof(float));
    }
    d->hidden = (float *)malloc(sizeof(float) * c->hidden);
    d->normed = (float *)malloc(sizeof(float) * c->hidden);
    d->query = (float *)malloc(sizeof(float) * qw);
    d->key = (float *)malloc(sizeof(float) * kvw);
    d->value = (float *)malloc(sizeof(float) * kvw);
    d->attention_out = (float *)malloc(sizeof(float) * qw);
    d->gate = (float *)malloc(sizeof(float) * c->ffn);
    d->up = (float *)malloc(sizeof(float) * c->ffn);
    return d;
}

void qwref_decoder_destroy(qwref_decoder *d) {
    if (!d) return;
    free_qmat(&d->embed);
    free_qmat(&d->lm_head);
    for (uint32_t l = 0; l < d->c.layers; ++l) {
        layer_mats *m = &d->layers[l];
        free_qmat(&m->q); free_qmat(&m->k); free_qmat(&m->v); free_qmat(&m->o);
        free_qmat(&m->gate); free_qmat(&m->up); free_qmat(&m->down);
        free(m->attention_norm); free(m->ffn_norm); free(m->q_norm); free(m->k_norm);
    }
    free(d->layers);
    for (uint32_t b = 0; b < d->batch; ++b) {
        free(d->seqs[b].keys);
        free(d->seqs[b].values);
        free(d->seqs[b].logits);
    }
    free(d->seqs);
    free(d->final_norm); free(d->rope_cos); free(d->rope_sin);
    free(d->hidden); free(d->normed); free(d->query); free(d->key); free(d->value);
    free(d->attention_out); free(d->gate); free(d->up);
    free(d);
}

int32_t qwref_decoder_set_vector(qwref_decoder *d, uint32_t kind, uint32_t layer, const float *values,
                                 uint32_t count) {
    float *dst = NULL;
    uint32_t expect = 0;
    if (kind == QWREF_VEC_FINAL_NORM) {
        dst = d->final_norm;
        expect = d->c.hidden;
    } else {
        if (layer >= d->c.layers) return QWREF_INVALID_ARGUMENT;
        layer_mats *m = &d->layers[layer];
        switch (kind) {
        case QWREF_VEC_ATTENTION_NORM: dst = m->attention_norm; expect = d->c.hidden; break;
        case QWREF_VEC_Q_NORM: dst = m->q_norm; expect = d->c.head_dim; break;
        case QWREF_VEC_K_NORM: dst = m->k_norm; expect = d->c.head_dim; break;
        case QWREF_VEC_FFN_NORM: dst = m->ffn_norm; expect = d->c.hidden; break;
        default: return QWREF_INVALID_ARGUMENT;
        }
    }
    if (count != expect) return QWREF_SHAPE_MISMATCH;
    memcpy(dst, values, sizeof(float) * count);
    return QWREF_OK;
}

/* kernels.zig:182-206 Matrix.apply: the arm of the matrix's storage. */
static int32_t apply(const qmat *m, float *out, const float *x) {
    if (m->format == QWREF_F32) return qwref_linear_f32(out, x, (const float *)m->data, m->rows, m->cols, 1);
    if (m->format == QWREF_F16) return qwref_linear_f16(out, x, (const uint16_t *)m->data, m->rows, m->cols, 1);
    return qwref_linear_quantized(out, x, m->format, m->scales, m->scales_len, m->data, m->data_len,
                                  m->rows, m->cols, 1);
}

/* decoder.zig:68-106 `appendCacheRow`: a copy into the f32 cache
 * (:77-83), or quantizeRow(.q8) into the q8 planes (:85-105). */
static void append_cache_row(qwref_decoder *d, sequence_state *s, uint32_t layer, uint32_t position,
                             const float *key, const float *value) {
    uint32_t kvw = d->c.kv_heads * d->c.head_dim;
    size_t layer_offset = (size_t)layer * d->cache_stride;
    if (d->cache_format == QWREF_CACHE_F32) {
        size_t offset = layer_offset + (size_t)position * kvw * sizeof(float);
        memcpy(s->keys + offset, key, sizeof(float) * kvw);
        memcpy(s->values + offset, value, sizeof(float) * kvw);
        return;
    }
    size_t scale_bytes = (size_t)(kvw / QWREF_GROUP) * 2u;
    size_t scale_offset = layer_offset + (size_t)position * scale_bytes;
    size_t code_offset = layer_offset + d->cache_scales + (size_t)position * kvw;
    qwref_quantize_row(QWREF_Q8, key, kvw, s->keys + scale_offset, s->keys + code_offset);
    qwref_quantize_row(QWREF_Q8, value, kvw, s->values + scale_offset, s->values + code_offset);
}

int32_t qwref_decoder_prefill_random(qwref_decoder *d, uint32_t seq, uint32_t count) {
    if (seq >= d->batch) return QWREF_INVALID_ARGUMENT;
    if (count > d->c.max_positions) return QWREF_LIMIT_EXCEEDED;
    sequence_state *s = &d->seqs[seq];
    uint32_t kvw = d->c.kv_heads * d->c.head_dim;
    float *rows_k = (float *)malloc(sizeof(float) * ((size_t)count * kvw + 1));
    float *rows_v = (float *)malloc(sizeof(float) * ((size_t)count * kvw + 1));
    for (uint32_t l = 0; l < d->c.layers; ++l) {
        uint32_t stream = STREAM_CACHE_BASE + 0x100 * seq + 2 * l;
        qwref_fill_normal(rows_k, (uint64_t)count * kvw, d->seed, stream, 1.0f);
        qwref_fill_normal(rows_v, (uint64_t)count * kvw, d->seed, stream + 1, 1.0f);
        for (uint32_t p = 0; p < count; ++p)
            append_cache_row(d, s, l, p, rows_k + (size_t)p * kvw, rows_v + (size_t)p * kvw);
    }
    free(rows_k);
    free(rows_v);
    s->position = count;
    return QWREF_OK;
}

/* decoder.zig:346-376 `embeddingRow` (quantized branch): the row
 * dequantized in the matrix's own format. */
/* decoder.zig:346-376 `embeddingRow`: f32 rows copied, f16 rows widened
 * (half_float.fromF16), quantized rows dequantized (quant.dequantizeRow).
 * A row past the end is refused. */
int32_t qwref_embedding_row(int32_t format, const uint8_t *scales, const uint8_t *data, uint32_t rows,
                            uint32_t cols, uint32_t row, float *out) {
    if (row >= rows) return QWREF_SHAPE_MISMATCH;
    if (format == QWREF_F32) {
        memcpy(out, data + (size_t)row * cols * 4u, sizeof(float) * cols);
        return QWREF_OK;
    }
    if (format == QWREF_F16) {
        const uint16_t *bits = (const uint16_t *)data + (size_t)row * cols;
        for (uint32_t i = 0; i < cols; ++i) out[i] = qwref_from_f16(bits[i]);
        return QWREF_OK;
    }
    if (qwref_data_bytes_per_group(format) == 0) return QWREF_UNSUPPORTED;
    if (cols % QWREF_GROUP != 0) return QWREF_SHAPE_MISMATCH;
    uint32_t gpr = cols / QWREF_GROUP;
    size_t data_row = (size_t)gpr * (size_t)qwref_data_bytes_per_group(format);
    qwref_dequantize_row(format, scales + (size_t)row * gpr * 2, data + (size_t)row * data_row, out, cols);
    return QWREF_OK;
}

static int32_t embedding_row(const qmat *m, uint32_t row, float *out) {
    return qwref_embedding_row(m->format, m->scales, m->data, m->rows, m->cols, row, out);
}

/* decoder.zig:133-287 `forwardToken`; with an audio row (:133-150) the row
 * replaces the token embedding (the projected audio features spliced into a
 * placeholder position) and everything after the embedding is the same
 * step. */
int32_t qwref_decoder_forward_row(qwref_decoder *d, uint32_t seq, uint32_t token, const float *audio_row,
                                  int32_t want_logits);

int32_t qwref_decoder_forward(qwref_decoder *d, uint32_t seq, uint32_t token, int32_t want_logits) {
    return qwref_decoder_forward_row(d, seq, token, NULL, want_logits);
}

int32_t qwref_decoder_forward_row(qwref_decoder *d, uint32_t seq, uint32_t token, const float *audio_row,
                                  int32_t want_logits) {
    if (seq >= d->batch) return QWREF_INVALID_ARGUMENT;
    const qwref_decoder_config *c = &d->c;
    sequence_state *s = &d->seqs[seq];
    if (s->position >= c->max_positions) return QWREF_LIMIT_EXCEEDED;
    uint32_t hs = c->hidden;
    if (audio_row) {
        memcpy(d->hidden, audio_row, sizeof(float) * hs);
    } else {
        int32_t status = embedding_row(&d->embed, token, d->hidden);
        if (status) return status;
    }
    uint32_t position = s->position;
    for (uint32_t l = 0; l < c->layers; ++l) {
        layer_mats *m = &d->layers[l];
        /* :165-172 rmsNormInto(attention_norm) */
        memcpy(d->normed, d->hidden, sizeof(float) * hs);
        qwref_rms_norm(d->normed, m->attention_norm, hs, 1, c->eps);
        /* :174-176 */
        apply(&m->q, d->query, d->normed);
        apply(&m->k, d->key, d->normed);
        apply(&m->v, d->value, d->normed);
        /* :180-193 per-head norm (q_norm, k_norm) before the rotation */
        qwref_rms_norm(d->query, m->q_norm, c->head_dim, c->heads, c->eps);
        qwref_rms_norm(d->key, m->k_norm, c->head_dim, c->kv_heads, c->eps);
        /* :195-214 */
        qwref_rope_in_place(d->query, &position, 1, c->heads, c->head_dim, d->rope_cos, d->rope_sin,
                            c->head_dim / 2);
        qwref_rope_in_place(d->key, &position, 1, c->kv_heads, c->head_dim, d->rope_cos, d->rope_sin,
                            c->head_dim / 2);
        /* :216 */
        append_cache_row(d, s, l, position, d->key, d->value);
        /* :220-253 */
        size_t lo = (size_t)l * d->cache_stride;
        if (d->cache_format == QWREF_CACHE_F32) {
            qwref_decode_attention_step(d->attention_out, d->query, (const float *)(s->keys + lo),
                                        (const float *)(s->values + lo), position + 1, c->heads, c->kv_heads,
                                        c->head_dim);
        } else {
            qwref_decode_attention_step_q8(d->attention_out, d->query, s->keys + lo,
                                           s->keys + lo + d->cache_scales, s->values + lo,
                                           s->values + lo + d->cache_scales, position + 1, c->heads,
                                           c->kv_heads, c->head_dim);
        }
        /* :256-257 */
        apply(&m->o, d->normed, d->attention_out);
        qwref_add_in_place(d->hidden, d->normed, hs);
        /* :259-271 rmsNormInto(ffn_norm) */
        memcpy(d->normed, d->hidden, sizeof(float) * hs);
        qwref_rms_norm(d->normed, m->ffn_norm, hs, 1, c->eps);
        apply(&m->gate, d->gate, d->normed);
        apply(&m->up, d->up, d->normed);
        qwref_silu_mul(d->gate, d->gate, d->up, c->ffn);
        apply(&m->down, d->normed, d->gate);
        qwref_add_in_place(d->hidden, d->normed, hs);
    }
    s->position += 1;
    if (!want_logits) return QWREF_OK;
    /* :277-286 rmsNormInto(final norm), output projection */
    memcpy(d->normed, d->hidden, sizeof(float) * hs);
    qwref_rms_norm(d->normed, d->final_norm, hs, 1, c->eps);
    apply(&d->lm_head, s->logits, d->normed);
    return QWREF_OK;
}

const float *qwref_decoder_logits(qwref_decoder *d, uint32_t seq) {
    return seq < d->batch ? d->seqs[seq].logits : NULL;
}

uint32_t qwref_decoder_position(qwref_decoder *d, uint32_t seq) {
    return seq < d->batch ? d->seqs[seq].position : 0;
}

/* decoder.zig:336-339 `step`. */
int32_t qwref_decoder_step(qwref_decoder *d, uint32_t seq, uint32_t token, uint32_t *next_token) {
    int32_t status = qwref_decoder_forward(d, seq, token, 1);
    if (status) return status;
    *next_token = qwref_argmax(d->seqs[seq].logits, d->c.vocab);
    return QWREF_OK;
}

static uint64_t hash_qmat(const qmat *m, uint64_t h) {
    h = qwref_fnv1a64(m->scales, m->scales_len, h);
    return qwref_fnv1a64(m->data, m->data_len, h);
}

uint64_t qwref_decoder_weights_hash(qwref_decoder *d) {
    uint64_t h = 0xcbf29ce484222325ull;
    h = hash_qmat(&d->embed, h);
    for (uint32_t l = 0; l < d->c.layers; ++l) {
        layer_mats *m = &d->layers[l];
        h = hash_qmat(&m->q, h); h = hash_qmat(&m->k, h); h = hash_qmat(&m->v, h);
        h = hash_qmat(&m->o, h); h = hash_qmat(&m->gate, h); h = hash_qmat(&m->up, h);
        h = hash_qmat(&m->down, h);
    }
    return hash_qmat(&d->lm_head, h);
}

/* One cache row of a layer as the decoder holds it (decoder.zig:58-65):
 * q8: the row's f16 key scales, its key codes, then the same for the values;
 * f32: the key row then the value row. Returns the bytes written to `out`,
 * 0 for a bad argument or a too small `capacity`. */
uint64_t qwref_decoder_cache_row(qwref_decoder *d, uint32_t seq, uint32_t layer, uint32_t position, uint8_t *out,
                                 uint64_t capacity) {
    if (seq >= d->batch || layer >= d->c.layers || position >= d->c.max_positions) return 0;
    const uint32_t kvw = d->c.kv_heads * d->c.head_dim;
    const size_t layer_offset = (size_t)layer * d->cache_stride;
    const sequence_state *s = &d->seqs[seq];
    if (d->cache_format == QWREF_CACHE_F32) {
        const size_t row = (size_t)kvw * sizeof(float);
        if (capacity < 2 * row) return 0;
        memcpy(out, s->keys + layer_offset + (size_t)position * row, row);
        memcpy(out + row, s->values + layer_offset + (size_t)position * row, row);
        return 2 * row;
    }
    const size_t scale_bytes = (size_t)(kvw / QWREF_GROUP) * 2u;
    const size_t scale_offset = layer_offset + (size_t)position * scale_bytes;
    const size_t code_offset = layer_offset + d->cache_scales + (size_t)position * kvw;
    if (capacity < 2 * (scale_bytes + kvw)) return 0;
    const uint8_t *planes[2] = {s->keys, s->values};
    for (int kv = 0; kv < 2; ++kv) {
        uint8_t *dst = out + kv * (scale_bytes + kvw);
        memcpy(dst, planes[kv] + scale_offset, scale_bytes);
        memcpy(dst + scale_bytes, planes[kv] + code_offset, kvw);
    }
    return 2 * (scale_bytes + kvw);
}

/* The inverse of qwref_decoder_cache_row: stores `len` bytes in that layout
 * as the row `position` of a layer. Test plumbing (no decoder.zig
 * counterpart): a checker writes another implementation's cache rows here,
 * so the next forward reads exactly those rows. Returns 0, or
 * QWREF_INVALID_ARGUMENT for a bad argument or a wrong length. */
int32_t qwref_decoder_set_cache_row(qwref_decoder *d, uint32_t seq, uint32_t layer, uint32_t position,
                                    const uint8_t *row, uint64_t len) {
    if (seq >= d->batch || layer >= d->c.layers || position >= d->c.max_positions) return QWREF_INVALID_ARGUMENT;
    const uint32_t kvw = d->c.kv_heads * d->c.head_dim;
    const size_t layer_offset = (size_t)layer * d->cache_stride;
    sequence_state *s = &d->seqs[seq];
    if (d->cache_format == QWREF_CACHE_F32) {
        const size_t bytes = (size_t)kvw * sizeof(float);
        if (len != 2 * bytes) return QWREF_INVALID_ARGUMENT;
        memcpy(s->keys + layer_offset + (size_t)position * bytes, row, bytes);
        memcpy(s->values + layer_offset + (size_t)position * bytes, row + bytes, bytes);
        return QWREF_OK;
    }
    const size_t scale_bytes = (size_t)(kvw / QWREF_GROUP) * 2u;
    if (len != 2 * (scale_bytes + kvw)) return QWREF_INVALID_ARGUMENT;
    uint8_t *planes[2] = {s->keys, s->values};
    for (int kv = 0; kv < 2; ++kv) {
        const uint8_t *src = row + kv * (scale_bytes + kvw);
        memcpy(planes[kv] + layer_offset + (size_t)position * scale_bytes, src, scale_bytes);
        memcpy(planes[kv] + layer_offset + d->cache_scales + (size_t)position * kvw, src + scale_bytes, kvw);
    }
    return QWREF_OK;
}

/* Sets a sequence's position (the next forward writes cache row `position`
 * and attends to the rows below it). Test plumbing, as above. */
int32_t qwref_decoder_set_position(qwref_decoder *d, uint32_t seq, uint32_t position) {
    if (seq >= d->batch) return QWREF_INVALID_ARGUMENT;
    if (position > d->c.max_positions) return QWREF_LIMIT_EXCEEDED;
    d->seqs[seq].position = position;
    return QWREF_OK;
}

uint64_t qwref_decoder_cache_hash(qwref_decoder *d, uint32_t seq) {
    if (seq >= d->batch) return 0;
    uint64_t h = 0xcbf29ce484222325ull;
    h = qwref_fnv1a64(d->seqs[seq].keys, (uint64_t)d->c.layers * d->cache_stride, h);
    return qwref_fnv1a64(d->seqs[seq].values, (uint64_t)d->c.layers * d->cache_stride, h);
}
