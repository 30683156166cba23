// Batch-1 (and small-batch) decode GEMV over the reference's packed planes.
//
// kernels.zig:118-158 linearQuantized with tokens small. The reference
// dequantizes a row into f32 scratch and dots it with the activations; here a
// row's codes are streamed once from HBM with 128-bit loads and multiplied in
// registers without ever forming a dequantized weight:
//
//   q4: the activations are first written as signed hex digit planes (see
//       device.h); each 16-byte load of codes holds 32 weights, XOR 0x8 turns
//       every biased nibble u into the signed code u - 8, and six
//       v_dot8_i32_i4 chains per dword give exact integer dot products
//       against the six digit planes. The integers are combined in f32 and
//       scaled by the group's f16 scale times the chunk's power-of-two
//       activation multiplier.
//   q8: each 16-byte load holds 16 codes, converted to f32 (exact) and
//       multiplied with f32 activations.
//
// Lane mapping: a wavefront owns RG consecutive rows (a "row group") at a
// time, and lane l always handles the same 16-byte column slices of those
// rows (slots s = 0..S-1 of the row group's flat slice list), so its
// activation operands stay in registers for the whole kernel while the wave
// walks row groups. U row groups are loaded per iteration to keep several
// 128-bit loads in flight per lane; the U*RG row sums are then reduced with
// one transposed butterfly across the wavefront.
#include "common.h"
#include "device.h"

namespace qwh {
namespace {

constexpr int kWave = 64;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// 128-bit streaming load (weights are read once per call: no reuse to keep).
__device__ __forceinline__ uint4 load_stream16(const void *p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

template <int V>
struct Log2 {
    static constexpr int value = 1 + Log2<V / 2>::value;
};
template <>
struct Log2<1> {
    static constexpr int value = 0;
};

// Sums acc[0..V) over the 64 lanes. Afterwards lane l holds the total of
// index (l >> (6 - log2 V)) in acc[0].
template <int V>
__device__ __forceinline__ void butterfly_reduce(float (&acc)[V], int lane) {
    constexpr int log_v = Log2<V>::value;
#pragma unroll
    for (int step = 0; step < log_v; ++step) {
        const int width = V >> step;
        const int mask = 32 >> step;
        const bool upper = (lane & mask) != 0;
#pragma unroll
        for (int i = 0; i < width / 2; ++i) {
            const float send = upper ? acc[i] : acc[i + width / 2];
            const float keep = upper ? acc[i + width / 2] : acc[i];
            acc[i] = keep + __shfl_xor(send, mask, kWave);
        }
    }
#pragma unroll
    for (int mask = 32 >> log_v; mask >= 1; mask >>= 1) acc[0] += __shfl_xor(acc[0], mask, kWave);
}

// ---------------------------------------------------------------------------
// Digit planes of the activations: one thread per 8 consecutive values, four
// threads per 32-value chunk.
// Layout: words[(t * T + c) * 24 + plane * 4 + q], mult[t * T + c].
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void prep_q4_kernel(const float *x, uint32_t total8,
                                                      uint32_t *words, float *mult) {
    const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
    const bool valid = gid < total8;
    float v[8];
    if (valid) {
        const float4 a = reinterpret_cast<const float4 *>(x)[gid * 2];
        const float4 b = reinterpret_cast<const float4 *>(x)[gid * 2 + 1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = 0.0f;
    }
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) amax = fmaxf(amax, fabsf(v[k]));
    amax = fmaxf(amax, __shfl_xor(amax, 1, kWave));
    amax = fmaxf(amax, __shfl_xor(amax, 2, kWave));
    const int e = dev::chunk_exponent(amax);
    uint32_t planes[6];
    dev::encode_digits8(v, e, planes);
    if (valid) {
        const uint32_t chunk = gid >> 2;
        const uint32_t q = gid & 3u;
        uint32_t *dst = words + (size_t)chunk * dev::kChunkWords + q;
#pragma unroll
        for (int j = 0; j < 6; ++j) dst[j * 4] = planes[j];
        if (q == 0) mult[chunk] = __builtin_ldexpf(1.0f, e - 22);
    }
}

// Exact integer dot products of one 16-byte slice of q4 codes (32 weights)
// against the six digit planes of its activations, combined in f32:
// returns sum_k (u_k - 8) * x_int_k with one rounding.
__device__ __forceinline__ float q4_slice_dot(const uint4 codes, const uint32_t (&d)[24]) {
    const int c0 = (int)(codes.x ^ 0x88888888u);
    const int c1 = (int)(codes.y ^ 0x88888888u);
    const int c2 = (int)(codes.z ^ 0x88888888u);
    const int c3 = (int)(codes.w ^ 0x88888888u);
    int I[6];
#pragma unroll
    for (int j = 0; j < 6; ++j) {
        int acc = __builtin_amdgcn_sdot8(c0, (int)d[j * 4 + 0], 0, false);
        acc = __builtin_amdgcn_sdot8(c1, (int)d[j * 4 + 1], acc, false);
        acc = __builtin_amdgcn_sdot8(c2, (int)d[j * 4 + 2], acc, false);
        acc = __builtin_amdgcn_sdot8(c3, (int)d[j * 4 + 3], acc, false);
        I[j] = acc;
    }
    // |I_j| <= 32 * 8 * 8, so both three-digit partial sums are exact in i32
    // and in f32.
    const int hi = (I[5] * 16 + I[4]) * 16 + I[3];
    const int lo = (I[2] * 16 + I[1]) * 16 + I[0];
    return fmaf((float)hi, 4096.0f, (float)lo);
}

struct GemvQ4Args {
    const uint32_t *words;  // digit planes, per token T * 24 words
    const float *mult;      // per token T multipliers
    const uint16_t *scales; // N * K/64
    const uint8_t *data;    // N * K/2
    float *out;             // tokens x N
    const float *residual;  // optional, tokens x N (may alias out)
    uint32_t n, k, t, row_groups;
};

template <int S, int RG, int U>
__global__ __launch_bounds__(256) void gemv_q4_kernel(const GemvQ4Args a) {
    constexpr int V = U * RG;
    const int lane = threadIdx.x & 63;
    const uint32_t wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const uint32_t nwaves = (gridDim.x * blockDim.x) >> 6;
    const uint32_t token = blockIdx.y;
    const uint32_t T = a.t;
    const uint32_t gpr = a.k >> 6;
    const size_t row_bytes = a.k >> 1;

    int rrow[S];
    uint32_t chunk[S];
    uint32_t D[S][24];
    float m[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const uint32_t f = (uint32_t)lane + 64u * s;
        rrow[s] = (int)(f / T);
        chunk[s] = f - (uint32_t)rrow[s] * T;
        const uint4 *src = reinterpret_cast<const uint4 *>(a.words + ((size_t)token * T + chunk[s]) * 24);
#pragma unroll
        for (int j = 0; j < 6; ++j) {
            const uint4 w = src[j];
            D[s][j * 4 + 0] = w.x;
            D[s][j * 4 + 1] = w.y;
            D[s][j * 4 + 2] = w.z;
            D[s][j * 4 + 3] = w.w;
        }
        m[s] = a.mult[(size_t)token * T + chunk[s]];
    }

    const uint32_t units = (a.row_groups + U - 1) / U;
    float *out = a.out + (size_t)token * a.n;
    const float *residual = a.residual ? a.residual + (size_t)token * a.n : nullptr;
    for (uint32_t unit = wave; unit < units; unit += nwaves) {
        uint4 code[U][S];
        uint16_t sc[U][S];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t rg = unit * U + u;
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const uint32_t row = rg * RG + rrow[s];
                if (rg < a.row_groups && row < a.n) {
                    code[u][s] = load_stream16(a.data + row * row_bytes + (size_t)chunk[s] * 16);
                    sc[u][s] = a.scales[(size_t)row * gpr + (chunk[s] >> 1)];
                } else {
                    code[u][s] = make_uint4(0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u);
                    sc[u][s] = 0;
                }
            }
        }
        float acc[V];
#pragma unroll
        for (int i = 0; i < V; ++i) acc[i] = 0.0f;
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const float val = q4_slice_dot(code[u][s], D[s]) * (dev::f16_bits_to_f32(sc[u][s]) * m[s]);
                if (RG == 1) {
                    acc[u] += val;
                } else {
#pragma unroll
                    for (int r = 0; r < RG; ++r) acc[u * RG + r] += (rrow[s] == r) ? val : 0.0f;
                }
            }
        }
        butterfly_reduce<V>(acc, lane);
        constexpr int lanes_per_value = 64 / V;
        if ((lane & (lanes_per_value - 1)) == 0) {
            const int idx = lane / lanes_per_value;
            const uint32_t rg = unit * U + idx / RG;
            const uint32_t row = rg * RG + idx % RG;
            if (rg < a.row_groups && row < a.n) out[row] = (residual ? residual[row] : 0.0f) + acc[0];
        }
    }
}

// Any K (a multiple of 64): one wavefront per row, lanes stride over the
// row's 16-byte slices and read the digit planes from memory.
__global__ __launch_bounds__(256) void gemv_q4_generic_kernel(const GemvQ4Args a) {
    const int lane = threadIdx.x & 63;
    const uint32_t wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const uint32_t nwaves = (gridDim.x * blockDim.x) >> 6;
    const uint32_t token = blockIdx.y;
    const uint32_t T = a.t;
    const uint32_t gpr = a.k >> 6;
    const size_t row_bytes = a.k >> 1;
    float *out = a.out + (size_t)token * a.n;
    const float *residual = a.residual ? a.residual + (size_t)token * a.n : nullptr;
    for (uint32_t row = wave; row < a.n; row += nwaves) {
        float acc = 0.0f;
        for (uint32_t c = lane; c < T; c += 64) {
            const uint4 code = reinterpret_cast<const uint4 *>(a.data + row * row_bytes)[c];
            uint32_t d[24];
            const uint4 *src = reinterpret_cast<const uint4 *>(a.words + ((size_t)token * T + c) * 24);
#pragma unroll
            for (int j = 0; j < 6; ++j) {
                const uint4 w = src[j];
                d[j * 4 + 0] = w.x; d[j * 4 + 1] = w.y; d[j * 4 + 2] = w.z; d[j * 4 + 3] = w.w;
            }
            const float mult = a.mult[(size_t)token * T + c];
            acc += q4_slice_dot(code, d) * (dev::f16_bits_to_f32(a.scales[(size_t)row * gpr + (c >> 1)]) * mult);
        }
        acc = dev::wave_sum(acc);
        if (lane == 0) out[row] = (residual ? residual[row] : 0.0f) + acc;
    }
}

// ---------------------------------------------------------------------------
// q8: slices of 16 codes; the lane's activations (16 f32 per slot) stay in
// registers. Codes convert exactly to f32 and the bias is subtracted before
// the multiply, so each product is the reference's decoded weight times x up
// to the group scale, applied once per slice.
// ---------------------------------------------------------------------------
struct GemvQ8Args {
    const float *x;         // tokens x K
    const uint16_t *scales; // N * K/64
    const uint8_t *data;    // N * K
    float *out;
    const float *residual;
    uint32_t n, k, t, row_groups;  // t = K/16 slices per row
};

__device__ __forceinline__ float q8_slice_dot(const uint4 codes, const float (&x)[16]) {
    float acc = 0.0f;
    const uint32_t w[4] = {codes.x, codes.y, codes.z, codes.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const float c = (float)((w[i] >> (8 * b)) & 0xffu) - 128.0f;
            acc = fmaf(c, x[i * 4 + b], acc);
        }
    }
    return acc;
}

template <int S, int RG, int U>
__global__ __launch_bounds__(256) void gemv_q8_kernel(const GemvQ8Args a) {
    constexpr int V = U * RG;
    const int lane = threadIdx.x & 63;
    const uint32_t wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const uint32_t nwaves = (gridDim.x * blockDim.x) >> 6;
    const uint32_t token = blockIdx.y;
    const uint32_t T = a.t;
    const uint32_t gpr = a.k >> 6;
    int rrow[S];
    uint32_t slice[S];
    float X[S][16];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const uint32_t f = (uint32_t)lane + 64u * s;
        rrow[s] = (int)(f / T);
        slice[s] = f - (uint32_t)rrow[s] * T;
        const float4 *src = reinterpret_cast<const float4 *>(a.x + (size_t)token * a.k + slice[s] * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = src[i];
            X[s][i * 4 + 0] = v.x; X[s][i * 4 + 1] = v.y; X[s][i * 4 + 2] = v.z; X[s][i * 4 + 3] = v.w;
        }
    }
    const uint32_t units = (a.row_groups + U - 1) / U;
    float *out = a.out + (size_t)token * a.n;
    const float *residual = a.residual ? a.residual + (size_t)token * a.n : nullptr;
    for (uint32_t unit = wave; unit < units; unit += nwaves) {
        uint4 code[U][S];
        uint16_t sc[U][S];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t rg = unit * U + u;
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const uint32_t row = rg * RG + rrow[s];
                if (rg < a.row_groups && row < a.n) {
                    code[u][s] = load_stream16(a.data + (size_t)row * a.k + (size_t)slice[s] * 16);
                    sc[u][s] = a.scales[(size_t)row * gpr + (slice[s] >> 2)];
                } else {
                    code[u][s] = make_uint4(0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u);
                    sc[u][s] = 0;
                }
            }
        }
        float acc[V];
#pragma unroll
        for (int i = 0; i < V; ++i) acc[i] = 0.0f;
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const float val = q8_slice_dot(code[u][s], X[s]) * dev::f16_bits_to_f32(sc[u][s]);
                if (RG == 1) {
                    acc[u] += val;
                } else {
#pragma unroll
                    for (int r = 0; r < RG; ++r) acc[u * RG + r] += (rrow[s] == r) ? val : 0.0f;
                }
            }
        }
        butterfly_reduce<V>(acc, lane);
        constexpr int lanes_per_value = 64 / V;
        if ((lane & (lanes_per_value - 1)) == 0) {
            const int idx = lane / lanes_per_value;
            const uint32_t rg = unit * U + idx / RG;
            const uint32_t row = rg * RG + idx % RG;
            if (rg < a.row_groups && row < a.n) out[row] = (residual ? residual[row] : 0.0f) + acc[0];
        }
    }
}

__global__ __launch_bounds__(256) void gemv_q8_generic_kernel(const GemvQ8Args a) {
    const int lane = threadIdx.x & 63;
    const uint32_t wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const uint32_t nwaves = (gridDim.x * blockDim.x) >> 6;
    const uint32_t token = blockIdx.y;
    const uint32_t gpr = a.k >> 6;
    float *out = a.out + (size_t)token * a.n;
    const float *residual = a.residual ? a.residual + (size_t)token * a.n : nullptr;
    for (uint32_t row = wave; row < a.n; row += nwaves) {
        float acc = 0.0f;
        for (uint32_t c = lane; c < a.t; c += 64) {
            const uint4 code = reinterpret_cast<const uint4 *>(a.data + (size_t)row * a.k)[c];
            float x[16];
            const float4 *src = reinterpret_cast<const float4 *>(a.x + (size_t)token * a.k + c * 16);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 v = src[i];
                x[i * 4 + 0] = v.x; x[i * 4 + 1] = v.y; x[i * 4 + 2] = v.z; x[i * 4 + 3] = v.w;
            }
            acc += q8_slice_dot(code, x) * dev::f16_bits_to_f32(a.scales[(size_t)row * gpr + (c >> 2)]);
        }
        acc = dev::wave_sum(acc);
        if (lane == 0) out[row] = (residual ? residual[row] : 0.0f) + acc;
    }
}

uint32_t gcd_u32(uint32_t a, uint32_t b) {
    while (b) {
        const uint32_t t = a % b;
        a = b;
        b = t;
    }
    return a;
}

// Waves to launch: enough to cover every unit, capped at a few per SIMD.
unsigned grid_blocks(uint32_t units, int cus) {
    const uint32_t waves = units;
    uint32_t blocks = (waves + 3) / 4;
    const uint32_t cap = (uint32_t)(cus > 0 ? cus : 256) * 8;
    if (blocks > cap) blocks = cap;
    if (blocks == 0) blocks = 1;
    return blocks;
}

#define QWH_GEMV_CASE(KERNEL, S_, RG_, U_)                                                        \
    if (S == S_ && RG == RG_) {                                                                   \
        args.row_groups = (args.n + RG_ - 1) / RG_;                                               \
        const uint32_t units = (args.row_groups + U_ - 1) / U_;                                   \
        KERNEL<S_, RG_, U_><<<dim3(grid_blocks(units, cus), tokens), 256, 0, s>>>(args);          \
        return hipGetLastError();                                                                 \
    }

}  // namespace

size_t q4_digit_bytes(uint32_t tokens, uint32_t cols) {
    const size_t chunks = (size_t)tokens * (cols / 32);
    return chunks * dev::kChunkWords * 4 + chunks * 4 + 256;
}

hipError_t launch_prep_q4(hipStream_t s, const float *x, uint32_t tokens, uint32_t cols, void *digits) {
    const uint32_t total8 = tokens * (cols / 8);
    const size_t chunks = (size_t)tokens * (cols / 32);
    uint32_t *words = static_cast<uint32_t *>(digits);
    float *mult = reinterpret_cast<float *>(words + chunks * dev::kChunkWords);
    prep_q4_kernel<<<(total8 + 255) / 256, 256, 0, s>>>(x, total8, words, mult);
    return hipGetLastError();
}

hipError_t launch_gemv_q4(hipStream_t s, int cus, const void *digits, const Matrix &w, uint32_t tokens,
                          float *out, const float *residual) {
    GemvQ4Args args{};
    const uint32_t T = w.cols / 32;
    const size_t chunks = (size_t)tokens * T;
    args.words = static_cast<const uint32_t *>(digits);
    args.mult = reinterpret_cast<const float *>(args.words + chunks * dev::kChunkWords);
    args.scales = reinterpret_cast<const uint16_t *>(w.scales);
    args.data = w.data;
    args.out = out;
    args.residual = residual;
    args.n = w.rows;
    args.k = w.cols;
    args.t = T;
    const uint32_t g = gcd_u32(T, 64);
    const uint32_t RG = 64 / g;
    const uint32_t S = T / g;
    QWH_GEMV_CASE(gemv_q4_kernel, 1, 1, 4)
    QWH_GEMV_CASE(gemv_q4_kernel, 1, 2, 4)
    QWH_GEMV_CASE(gemv_q4_kernel, 1, 4, 2)
    QWH_GEMV_CASE(gemv_q4_kernel, 1, 8, 1)
    QWH_GEMV_CASE(gemv_q4_kernel, 1, 16, 1)
    QWH_GEMV_CASE(gemv_q4_kernel, 1, 32, 1)
    QWH_GEMV_CASE(gemv_q4_kernel, 2, 1, 2)
    QWH_GEMV_CASE(gemv_q4_kernel, 3, 1, 2)
    QWH_GEMV_CASE(gemv_q4_kernel, 3, 2, 2)
    QWH_GEMV_CASE(gemv_q4_kernel, 3, 4, 1)
    gemv_q4_generic_kernel<<<dim3(grid_blocks(w.rows, cus), tokens), 256, 0, s>>>(args);
    return hipGetLastError();
}

hipError_t launch_gemv_q8(hipStream_t s, int cus, const float *x, const Matrix &w, uint32_t tokens,
                          float *out, const float *residual) {
    GemvQ8Args args{};
    const uint32_t T = w.cols / 16;
    args.x = x;
    args.scales = reinterpret_cast<const uint16_t *>(w.scales);
    args.data = w.data;
    args.out = out;
    args.residual = residual;
    args.n = w.rows;
    args.k = w.cols;
    args.t = T;
    const uint32_t g = gcd_u32(T, 64);
    const uint32_t RG = 64 / g;
    const uint32_t S = T / g;
    QWH_GEMV_CASE(gemv_q8_kernel, 1, 1, 4)
    QWH_GEMV_CASE(gemv_q8_kernel, 1, 2, 4)
    QWH_GEMV_CASE(gemv_q8_kernel, 1, 4, 2)
    QWH_GEMV_CASE(gemv_q8_kernel, 1, 8, 1)
    QWH_GEMV_CASE(gemv_q8_kernel, 1, 16, 1)
    QWH_GEMV_CASE(gemv_q8_kernel, 2, 1, 2)
    QWH_GEMV_CASE(gemv_q8_kernel, 3, 1, 2)
    QWH_GEMV_CASE(gemv_q8_kernel, 3, 2, 2)
    gemv_q8_generic_kernel<<<dim3(grid_blocks(w.rows, cus), tokens), 256, 0, s>>>(args);
    return hipGetLastError();
}

}  // namespace qwh
