// Device-side helpers shared by the kernels: f16 codec, wave reductions,
// the bit-exact quantizer of one value, and the signed-hex-digit encoding of
// activations consumed by the q4 GEMV.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace qwh {
namespace dev {

constexpr int kWave = 64;

// v of lane (lane ^ MASK) for a compile-time MASK < 64, without a trip
// through LDS: DPP row permutes for 1, 2 (quad_perm), 4 (row_shr / row_shl
// by 4, picked by lane bit 2) and 8 (row_ror:8, which is xor 8 within a row
// of 16), and the gfx950 permlane swaps for 16 and 32 (each returns both
// halves; lane bit 4 or 5 picks the partner's).
template <int MASK>
__device__ __forceinline__ float xor_lane(float v) {
    static_assert(MASK == 1 || MASK == 2 || MASK == 4 || MASK == 8 || MASK == 16 || MASK == 32, "mask");
    const int x = __builtin_bit_cast(int, v);
    if constexpr (MASK == 1) {
        return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false));
    } else if constexpr (MASK == 2) {
        return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false));
    } else if constexpr (MASK == 4) {
        const int lane = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
        const int down = __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);  // lane - 4
        const int up = __builtin_amdgcn_update_dpp(0, x, 0x104, 0xF, 0xF, false);    // lane + 4
        return __builtin_bit_cast(float, (lane & 4) ? down : up);
    } else if constexpr (MASK == 8) {
        return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, false));
    } else if constexpr (MASK == 16) {
        const int lane = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
        const auto p = __builtin_amdgcn_permlane16_swap((unsigned)x, (unsigned)x, false, false);
        return __builtin_bit_cast(float, (lane & 16) ? p[0] : p[1]);
    } else {
        const int lane = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
        const auto p = __builtin_amdgcn_permlane32_swap((unsigned)x, (unsigned)x, false, false);
        return __builtin_bit_cast(float, (lane & 32) ? p[0] : p[1]);
    }
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, xor_lane<32>(v));
    v = fmaxf(v, xor_lane<16>(v));
    v = fmaxf(v, xor_lane<8>(v));
    v = fmaxf(v, xor_lane<4>(v));
    v = fmaxf(v, xor_lane<2>(v));
    return fmaxf(v, xor_lane<1>(v));
}

__device__ __forceinline__ float wave_sum(float v) {
    v += xor_lane<32>(v);
    v += xor_lane<16>(v);
    v += xor_lane<8>(v);
    v += xor_lane<4>(v);
    v += xor_lane<2>(v);
    return v + xor_lane<1>(v);
}

// The reference's erf (math.zig:46-60): the Numerical Recipes Chebyshev fit
// of erfc (`erfcc`), evaluated in f32 by Horner's rule.
__device__ __forceinline__ float erf_fit(float x) {
    const float magnitude = fabsf(x);
    const float t = 1.0f / (1.0f + 0.5f * magnitude);
    float poly = -0.82215223f + t * 0.17087277f;
    poly = 1.48851587f + t * poly;
    poly = -1.13520398f + t * poly;
    poly = 0.27886807f + t * poly;
    poly = -0.18628806f + t * poly;
    poly = 0.09678418f + t * poly;
    poly = 0.37409196f + t * poly;
    poly = 1.00002368f + t * poly;
    const float tau = t * expf(-magnitude * magnitude - 1.26551223f + t * poly);
    return copysignf(1.0f - tau, x);
}

__device__ __forceinline__ float gelu(float x) { return 0.5f * x * (1.0f + erf_fit(x * 0.70710678f)); }

// Sum over the lanes that differ from this one only in bits below N (N a
// power of two <= 64): an all-reduce within aligned groups of N lanes.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (N >= 64) v += xor_lane<32>(v);
    if constexpr (N >= 32) v += xor_lane<16>(v);
    if constexpr (N >= 16) v += xor_lane<8>(v);
    if constexpr (N >= 8) v += xor_lane<4>(v);
    if constexpr (N >= 4) v += xor_lane<2>(v);
    if constexpr (N >= 2) v += xor_lane<1>(v);
    return v;
}

// f32 -> f16 bits, round to nearest even, overflow to infinity
// (half_float.zig:14-17). Integer arithmetic only, so the result does not
// depend on the hardware rounding mode.
__device__ __forceinline__ uint16_t f32_to_f16_bits(float value) {
    uint32_t bits = __float_as_uint(value);
    uint32_t sign = (bits >> 16) & 0x8000u;
    int exponent = (int)((bits >> 23) & 0xffu);
    uint32_t mantissa = bits & 0x7fffffu;
    if (exponent == 0xff) return (uint16_t)(sign | 0x7c00u | (mantissa ? 0x200u : 0u));
    int half_exponent = exponent - 112;  // -127 + 15
    if (half_exponent >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    uint32_t shift;
    uint32_t base;
    if (half_exponent <= 0) {
        if (half_exponent < -10) return (uint16_t)sign;
        mantissa |= 0x800000u;
        shift = (uint32_t)(14 - half_exponent);
        base = 0;
    } else {
        shift = 13;
        base = (uint32_t)half_exponent << 10;
    }
    uint32_t kept = mantissa >> shift;
    uint32_t rest = mantissa & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    uint32_t rounded = kept + ((rest > half || (rest == half && (kept & 1u))) ? 1u : 0u);
    return (uint16_t)(sign | (base + rounded));
}

// f16 bits -> f32, exact (the hardware conversion keeps f16 subnormals).
__device__ __forceinline__ float f16_bits_to_f32(uint16_t bits) {
    return (float)__builtin_bit_cast(_Float16, bits);
}

// quant.zig:280-288 `quantizeOne`: round half away from zero against the
// stored scale, clamp to [min_code, max_code].
__device__ __forceinline__ int quantize_one(float value, float stored_scale, int min_code,
                                            int max_code) {
    if (stored_scale == 0.0f) return 0;
    float scaled = __fdiv_rn(value, stored_scale);
    float rounded = scaled >= 0.0f ? floorf(__fadd_rn(scaled, 0.5f)) : ceilf(__fsub_rn(scaled, 0.5f));
    if (rounded <= (float)min_code) return min_code;
    if (rounded >= (float)max_code) return max_code;
    return (int)rounded;
}

// ---------------------------------------------------------------------------
// Activation digits for the q4 GEMV.
//
// A chunk of 32 consecutive activations x_k is written as
//     x_k ~= m * sum_{j<6} d_{j,k} 16^j,   d in [-8, 7],   m = 2^(e-22),
// where 2^e bounds the chunk's largest |x|: x_int = rint(x * 2^(22-e)) is a
// 23-bit signed integer, and u = x_int + 0x888888 has hex digit j equal to
// d_j + 8. Digit plane j of 8 consecutive activations packs (d_j mod 16) into
// the 8 nibbles of one dword, in element order -- the order of the q4 code
// nibbles (quant.zig:36-41), so v_dot8_i32_i4 multiplies matching elements.
// A chunk is 6 planes x 4 dwords, plane major, followed by nothing: the
// per-chunk multiplier m lives in a separate f32 array.
// ---------------------------------------------------------------------------
constexpr int kDigitPlanes = 6;
constexpr int kChunk = 32;                       // activations per chunk
constexpr int kChunkWords = kDigitPlanes * 4;    // u32 per chunk

// Transposes an 8 x 8 matrix of nibbles held as 8 words (row k = word k,
// column j = nibble j): afterwards nibble k of w[j] is what nibble j of w[k]
// was. Three rounds swap the off-diagonal blocks of 16-bit, 8-bit and 4-bit
// width.
__device__ __forceinline__ void transpose_nibbles8(uint32_t (&w)[8]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t a = w[k], b = w[k + 4];
        w[k] = (a & 0x0000ffffu) | (b << 16);
        w[k + 4] = (a >> 16) | (b & 0xffff0000u);
    }
#pragma unroll
    for (int k = 0; k < 8; k += (k & 1) ? 3 : 1) {  // k = 0, 1, 4, 5
        const uint32_t a = w[k], b = w[k + 2];
        w[k] = (a & 0x00ff00ffu) | ((b & 0x00ff00ffu) << 8);
        w[k + 2] = ((a >> 8) & 0x00ff00ffu) | (b & 0xff00ff00u);
    }
#pragma unroll
    for (int k = 0; k < 8; k += 2) {
        const uint32_t a = w[k], b = w[k + 1];
        w[k] = (a & 0x0f0f0f0fu) | ((b & 0x0f0f0f0fu) << 4);
        w[k + 1] = ((a >> 4) & 0x0f0f0f0fu) | (b & 0xf0f0f0f0u);
    }
}

// Signed hex digits of x_int in nibbles 0..5: adding 0x888888 makes every
// digit d + 8 (no carries), and XOR 0x888888 turns d + 8 into d mod 16.
__device__ __forceinline__ uint32_t digit_word(float v, float up) {
    return (uint32_t)((int)__builtin_rintf(v * up) + 0x888888) ^ 0x888888u;
}

// Encodes 8 activations (this thread's dword column q of its chunk) given the
// chunk exponent e. Writes plane j of this column to planes[j].
__device__ __forceinline__ void encode_digits8(const float v[8], int e, uint32_t planes[6]) {
    const float up = __builtin_ldexpf(1.0f, 22 - e);
    uint32_t w[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) w[k] = digit_word(v[k], up);
    transpose_nibbles8(w);
#pragma unroll
    for (int j = 0; j < 6; ++j) planes[j] = w[j];
}

// Sum over a 256-thread workgroup; every thread gets the total (lds: 4
// floats, reused after the call).
__device__ __forceinline__ float block_sum_256(float v, float *lds) {
    v = wave_sum(v);
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) lds[wave] = v;
    __syncthreads();
    return (lds[0] + lds[1]) + (lds[2] + lds[3]);
}

// math.zig:99-116 layerNorm statistics of one row by a 256-thread workgroup:
// the mean, then the centred variance, then 1 / sqrt(variance + eps). A row
// value is then (x - mean) * inverse_std * weight + bias.
__device__ __forceinline__ void layer_norm_stats(const float *row, uint32_t width, float eps, float *lds,
                                                 float &mean, float &inverse_std) {
    float sum = 0.0f;
    for (uint32_t i = threadIdx.x; i < width; i += 256) sum += row[i];
    mean = block_sum_256(sum, lds) / (float)width;
    float squares = 0.0f;
    for (uint32_t i = threadIdx.x; i < width; i += 256) {
        const float centered = row[i] - mean;
        squares += centered * centered;
    }
    const float variance = block_sum_256(squares, lds) / (float)width;
    inverse_std = 1.0f / sqrtf(variance + eps);
}

// Exponent e with |x| <= 2^e for the chunk maximum `amax` (clamped so that
// 2^(22-e) stays finite; an all-zero chunk uses e = 0).
__device__ __forceinline__ int chunk_exponent(float amax) {
    if (!(amax > 0.0f)) return 0;
    int e;
    (void)__builtin_frexpf(amax, &e);  // amax = f 2^e, f in [0.5, 1)
    return e < -100 ? -100 : e;
}

}  // namespace dev
}  // namespace qwh
