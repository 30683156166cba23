// Device quantizer (quant.zig:197-288, bit exact) and the synthetic input
// generator used for random-init weights and key/value states.
#include "common.h"
#include "device.h"

namespace qwh {
namespace {

// ---------------------------------------------------------------------------
// Synthetic generator. Value i of stream `stream` under `seed`:
//   base  = seed + stream * 0x9e3779b9                       (mod 2^32)
//   draw n = mulberry32 output of state base + n * 0x6d2b79f5  (n >= 1)
//   u1, u2 = draws 2i+1, 2i+2
//   value = f32( sqrt(-2 ln(1 - u1/2^32)) * cos(2 pi u2/2^32) )
// mulberry32 and Box-Muller are those of the reference's seeded test inputs
// (tests/gpu/reference.mjs:35-58). ln, cos and sqrt are evaluated in double by
// fixed sequences of IEEE +, -, *, / (no fused operations: contraction is off
// in these functions), so every host and device that runs the same sequence
// gets the same bits.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t mulberry32_output(uint32_t state) {
    uint32_t value = state;
    value = (value ^ (value >> 15)) * (value | 1u);
    value = value ^ (value + (value ^ (value >> 7)) * (value | 61u));
    return value ^ (value >> 14);
}

// ln x for x in (0, 1]: x = m 2^e with m in (sqrt(1/2), sqrt(2)]; ln m = 2
// atanh(s), s = (m - 1)/(m + 1), odd series through s^23; ln 2 split in a
// high and a low part.
__device__ double det_log(double x) {
#pragma clang fp contract(off)
    unsigned long long bits = (unsigned long long)__double_as_longlong(x);
    int e = (int)((bits >> 52) & 0x7ffull) - 1023;
    double m = __longlong_as_double((long long)((bits & 0x000fffffffffffffull) | 0x3ff0000000000000ull));
    if (m > 1.4142135623730951) {
        m = m * 0.5;
        e = e + 1;
    }
    const double s = (m - 1.0) / (m + 1.0);
    const double z = s * s;
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
    const double log_m = (2.0 * s) * p;
    const double de = (double)e;
    return de * 6.93147180369123816490e-01 + (de * 1.90821492927058770002e-10 + log_m);
}

// cos(2 pi t), t in [0, 1): exact split of 4t into a quadrant and a fraction,
// reflection of the fraction into [0, 1/2], Taylor series of cos / sin of
// the angle (at most pi/4) through degree 20 / 21.
__device__ double det_cos2pi(double t) {
#pragma clang fp contract(off)
    const double q4 = t * 4.0;
    const int q = (int)q4;
    const double f = q4 - (double)q;
    int use_sin = q & 1;
    double g = f;
    if (f > 0.5) {
        g = 1.0 - f;
        use_sin = !use_sin;
    }
    const double y = g * 1.5707963267948966;
    const double y2 = y * y;
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

// sqrt y, y >= 0: a first guess from halving the exponent, six Newton steps.
__device__ double det_sqrt(double y) {
#pragma clang fp contract(off)
    if (y == 0.0) return 0.0;
    double g = __longlong_as_double(
        (long long)(((unsigned long long)__double_as_longlong(y) >> 1) + 0x1ff8000000000000ull));
    for (int i = 0; i < 6; ++i) g = 0.5 * (g + y / g);
    return g;
}

__device__ float synth_normal(uint32_t base, uint64_t index) {
#pragma clang fp contract(off)
    const uint32_t n1 = (uint32_t)(2 * index + 1);
    const uint32_t u1 = mulberry32_output(base + n1 * 0x6d2b79f5u);
    const uint32_t u2 = mulberry32_output(base + (n1 + 1u) * 0x6d2b79f5u);
    const double first = 1.0 - (double)u1 / 4294967296.0;
    const double second = (double)u2 / 4294967296.0;
    const double radius = det_sqrt(-2.0 * det_log(first));
    return (float)(radius * det_cos2pi(second));
}

__global__ void synth_normal_kernel(uint32_t base, uint64_t first, uint64_t count, float scale, float *out) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride)
        out[i] = synth_normal(base, first + i) * scale;
}

// ---------------------------------------------------------------------------
// quant.zig:197-278 quantizeRow / quantizeGroup. One wavefront per group of
// 64 values (groups are row major across rows, so a whole matrix is one flat
// list of groups): lane i quantizes value i. The group maximum is exact in
// any order; the scale is f16(max / bias) and the codes are computed against
// the stored scale, exactly as the reference.
// ---------------------------------------------------------------------------
template <int Format>
__global__ __launch_bounds__(256) void quantize_groups_kernel(const float *values, uint64_t groups,
                                                              uint8_t *scales, uint8_t *data) {
    constexpr int bias = Format == QWH_FORMAT_Q4 ? 8 : (Format == QWH_FORMAT_Q5 ? 16 : 128);
    constexpr int data_bytes = Format == QWH_FORMAT_Q4 ? 32 : (Format == QWH_FORMAT_Q5 ? 40 : 64);
    const int lane = threadIdx.x & 63;
    const uint64_t waves = ((uint64_t)gridDim.x * blockDim.x) >> 6;
    for (uint64_t g = (((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6); g < groups; g += waves) {
        const float v = values[g * 64 + lane];
        const float amax = dev::wave_max(fabsf(v));
        const uint16_t scale_bits = dev::f32_to_f16_bits(__fdiv_rn(amax, (float)bias));
        const float stored = dev::f16_bits_to_f32(scale_bits);
        const uint32_t u = (uint32_t)(dev::quantize_one(v, stored, -bias, bias - 1) + bias);
        uint8_t *codes = data + g * data_bytes;
        if (lane == 0) {
            scales[g * 2] = (uint8_t)(scale_bits & 0xff);
            scales[g * 2 + 1] = (uint8_t)(scale_bits >> 8);
        }
        if (Format == QWH_FORMAT_Q8) {
            codes[lane] = (uint8_t)u;
        } else {
            const uint32_t odd = __shfl_down(u & 0xfu, 1, 64);
            if ((lane & 1) == 0) codes[lane >> 1] = (uint8_t)((u & 0xfu) | (odd << 4));
            if (Format == QWH_FORMAT_Q5) {
                // quant.zig:265-267: weight j's fifth bit is bit j % 8 of byte 32 + j / 8.
                const uint64_t high = __ballot((u & 0x10u) != 0);
                if (lane < 8) codes[32 + lane] = (uint8_t)(high >> (8 * lane));
            }
        }
    }
}

}  // namespace

hipError_t launch_synth_normal(hipStream_t s, uint32_t seed, uint32_t stream, uint64_t first,
                               uint64_t count, float scale, float *out) {
    if (count == 0) return hipSuccess;
    const uint32_t base = seed + stream * 0x9e3779b9u;
    uint64_t blocks = (count + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    synth_normal_kernel<<<(unsigned)blocks, 256, 0, s>>>(base, first, count, scale, out);
    return hipGetLastError();
}

hipError_t launch_quantize_rows(hipStream_t s, int format, const float *values, uint64_t groups,
                                uint8_t *scales, uint8_t *data) {
    if (groups == 0) return hipSuccess;
    uint64_t blocks = (groups + 3) / 4;
    if (blocks > 65536) blocks = 65536;
    switch (format) {
    case QWH_FORMAT_Q4:
        quantize_groups_kernel<QWH_FORMAT_Q4><<<(unsigned)blocks, 256, 0, s>>>(values, groups, scales, data);
        break;
    case QWH_FORMAT_Q5:
        quantize_groups_kernel<QWH_FORMAT_Q5><<<(unsigned)blocks, 256, 0, s>>>(values, groups, scales, data);
        break;
    case QWH_FORMAT_Q8:
        quantize_groups_kernel<QWH_FORMAT_Q8><<<(unsigned)blocks, 256, 0, s>>>(values, groups, scales, data);
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace qwh
