// Small-batch q4 GEMV on the matrix cores: kernels.zig:118-158
// linearQuantized for 2 or more tokens (the decoder step at batch > 1).
//
// One v_mfma_i32_16x16x64_i8 multiplies 16 tokens by 16 weight rows over 64
// consecutive columns -- exactly one quantization group (quant.zig:49), so
// its integer result takes that group's single f16 scale per row. The
// operands are exact integers:
//   weights      the q4 codes u - 8 as signed bytes;
//   activations  per token and group, x_int = rint(x * 2^(22-e)) with 2^e
//                bounding the group's largest |x| (|x_int| <= 2^22), written
//                as three signed base-256 digit planes d0 + 256 d1 + 65536 d2
//                (d in [-128, 127]); one MFMA per plane.
// Each plane's dot product is below 2^16 in magnitude, so the int32 results
// are exact; they are combined in f32 and scaled by f16 scale * 2^(e-22).
//
// Operand layout. Lane l of a wavefront feeds token (or weight row) l % 16
// and the 16 columns 16 * (l / 16) .. +15 of the group. A lane's 16 codes are
// 8 bytes of the row (two per byte, even column in the low nibble,
// quant.zig:36-41); nibble masks split them into the bytes of columns
// {0,2,4,6}, {1,3,5,7}, {8,10,12,14}, {9,11,13,15}. The activation digits are
// stored in that same order, so byte b of both operands belongs to the same
// column. Layout of the digits, per 16-token tile and group:
//   digits[tile][g][plane][token 0..15][64 bytes],  mult[tile][g][16] f32.
//
// Work split: a workgroup owns TILES 16-row tiles of the output (1, 2 or 4,
// by the row count) for one 16-token tile; its four wavefronts take
// consecutive quarters of the groups and their partial sums are added in
// wavefront order through LDS (deterministic).
#include "common.h"
#include "device.h"

namespace qwh {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kTokenTile = 16;
constexpr int kRowTile = 16;
constexpr int kPlaneBytes = kTokenTile * 64;           // one digit plane of a group
constexpr int kGroupBytes = 3 * kPlaneBytes;            // three planes
constexpr int kStage = 4;                               // groups per pipeline stage

// Signed-byte codes of 8 packed q4 bytes (16 codes), in the column order
// described above: (nibble + 0x78) ^ 0x80 = nibble - 8 as a two's complement
// byte, with no carry between bytes.
__device__ __forceinline__ v4i expand_q4(uint2 w) {
    v4i b;
    b.x = (int)(((w.x & 0x0f0f0f0fu) + 0x78787878u) ^ 0x80808080u);
    b.y = (int)((((w.x >> 4) & 0x0f0f0f0fu) + 0x78787878u) ^ 0x80808080u);
    b.z = (int)(((w.y & 0x0f0f0f0fu) + 0x78787878u) ^ 0x80808080u);
    b.w = (int)((((w.y >> 4) & 0x0f0f0f0fu) + 0x78787878u) ^ 0x80808080u);
    return b;
}

struct BatchArgs {
    const uint8_t *digits;   // [token tiles][groups][3][16][64]
    const float *mult;       // [token tiles][groups][16]
    const uint16_t *scales;  // N * K/64
    const uint8_t *data;     // N * K/2
    float *out;              // tokens x N, or tokens x N/2 with pairs
    const float *residual;   // optional, tokens x N (may alias out); not with pairs
    uint32_t n, k, tokens;
    uint32_t pairs;          // rows 2j, 2j+1 are gate_j, up_j: write silu(gate_j) * up_j
};

// siluMul of one gate / up pair (math.zig:69-71: silu(g) = g / (1 + exp(-g))).
__device__ __forceinline__ float silu_mul(float g, float u) {
    return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, expf(-g))), u);
}

// Groups per pipeline stage: fewer when a wave has more tiles (registers).
template <int TILES>
constexpr int stage_groups() { return TILES >= 4 ? 2 : kStage; }

template <int TILES>
struct Stage {
    static constexpr int G = stage_groups<TILES>();
    v4i a[G][3];
    uint2 w[G][TILES];
    uint16_t s[G][TILES];
    float4 m[G];
};

// TILES 16-row tiles per wavefront: the activation digits of a group, loaded
// once, feed TILES x 3 MFMAs.
template <int TILES>
__global__ __launch_bounds__(256) void gemv_q4_batch_kernel(const BatchArgs a) {
    constexpr int ROWS = kRowTile * TILES;  // rows of the workgroup (and of each wave)
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int col = lane & 15;     // weight row within a tile / token within the token tile
    const int blk = lane >> 4;     // 16-column block of the group
    const uint32_t gpr = a.k >> 6;
    const uint32_t tile = blockIdx.y;
    const uint32_t row0 = blockIdx.x * ROWS;
    const uint32_t g0 = wave * gpr / 4;
    const uint32_t g1 = (wave + 1) * gpr / 4;
    const uint8_t *wrow[TILES];
    const uint16_t *srow[TILES];
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
        uint32_t row = row0 + t * kRowTile + col;
        if (row >= a.n) row = a.n - 1;  // loads stay in the matrix; the store is skipped
        wrow[t] = a.data + (size_t)row * (a.k >> 1) + blk * 8;
        srow[t] = a.scales + (size_t)row * gpr;
    }
    const uint8_t *dig = a.digits + (size_t)tile * gpr * kGroupBytes + col * 64 + blk * 16;
    const float *mul = a.mult + (size_t)tile * gpr * kTokenTile + blk * 4;

    constexpr int G = stage_groups<TILES>();
    auto load = [&](Stage<TILES> &st, uint32_t g) {
#pragma unroll
        for (int i = 0; i < G; ++i) {
            const uint32_t gi = g + i < g1 ? g + i : g1 - 1;  // clamped: no branch in the stage
#pragma unroll
            for (int t = 0; t < TILES; ++t) {
                st.w[i][t] = *reinterpret_cast<const uint2 *>(wrow[t] + (size_t)gi * 32);
                st.s[i][t] = srow[t][gi];
            }
            st.m[i] = *reinterpret_cast<const float4 *>(mul + (size_t)gi * kTokenTile);
#pragma unroll
            for (int p = 0; p < 3; ++p)
                st.a[i][p] = *reinterpret_cast<const v4i *>(dig + (size_t)gi * kGroupBytes + p * kPlaneBytes);
        }
    };
    // Wave 0 writes the tiles: its residuals are fetched now, with the first
    // weights, rather than after the reduction.
    float res[TILES][4] = {};
    if (wave == 0 && a.residual) {
#pragma unroll
        for (int t = 0; t < TILES; ++t) {
            const uint32_t out_row = row0 + t * kRowTile + col;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t tok = tile * kTokenTile + blk * 4 + r;
                if (out_row < a.n && tok < a.tokens) res[t][r] = a.residual[(size_t)tok * a.n + out_row];
            }
        }
    }
    float acc[TILES][4] = {};
    auto process = [&](const Stage<TILES> &st, uint32_t g) {
#pragma unroll
        for (int i = 0; i < G; ++i) {
            if (g + i >= g1) break;
            const float m[4] = {st.m[i].x, st.m[i].y, st.m[i].z, st.m[i].w};
#pragma unroll
            for (int t = 0; t < TILES; ++t) {
                const v4i b = expand_q4(st.w[i][t]);
                const v4i zero = {0, 0, 0, 0};
                const v4i d0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(st.a[i][0], b, zero, 0, 0, 0);
                const v4i d1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(st.a[i][1], b, zero, 0, 0, 0);
                const v4i d2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(st.a[i][2], b, zero, 0, 0, 0);
                const float s = dev::f16_bits_to_f32(st.s[i][t]);
                const int p0[4] = {d0.x, d0.y, d0.z, d0.w};
                const int p1[4] = {d1.x, d1.y, d1.z, d1.w};
                const int p2[4] = {d2.x, d2.y, d2.z, d2.w};
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float f = (float)(p0[r] + p1[r] * 256) + 65536.0f * (float)p2[r];
                    acc[t][r] = fmaf(f, s * m[r], acc[t][r]);
                }
            }
        }
    };

    if (g0 < g1) {
        Stage<TILES> A, B;
        load(A, g0);
        uint32_t g = g0;
        for (; g + G < g1; g += 2 * G) {
            load(B, g + G);
            process(A, g);
            load(A, g + 2 * G < g1 ? g + 2 * G : g);
            process(B, g + G);
        }
        if (g < g1) process(A, g);
    }

    // Lane l holds tokens 4 * (l / 16) + r of weight row l % 16 of each tile.
    __shared__ float part[4][TILES][4][64];
#pragma unroll
    for (int t = 0; t < TILES; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) part[wave][t][r][lane] = acc[t][r];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
        const uint32_t out_row = row0 + t * kRowTile + col;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t tok = tile * kTokenTile + blk * 4 + r;
            const float total =
                ((part[0][t][r][lane] + part[1][t][r][lane]) + part[2][t][r][lane]) + part[3][t][r][lane];
            if (a.pairs) {
                // Row + 1 is the next lane's row (same token).
                const float partner = __shfl_down(total, 1, 64);
                if (tok < a.tokens && (out_row & 1u) == 0 && out_row < a.n)
                    a.out[(size_t)tok * (a.n / 2) + (out_row >> 1)] = silu_mul(total, partner);
            } else if (tok < a.tokens && out_row < a.n) {
                a.out[(size_t)tok * a.n + out_row] = res[t][r] + total;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Activation digits. One workgroup per token (padding tokens write zeros);
// thread i takes 8 consecutive values 8i .. 8i+7 of each 2048-value stretch,
// so the 8 threads of a group are consecutive lanes. Forms as in the q4 GEMV:
// f32 values as they are, or RMSNorm (math.zig:120-130).
// ---------------------------------------------------------------------------
enum class Prep : int { F32 = 0, RmsNorm = 1 };

struct PrepArgs {
    const float *x;      // tokens x K
    const float *norm;   // RmsNorm weights
    float eps;
    uint32_t k, tokens;
    uint8_t *digits;
    float *mult;
};

__device__ __forceinline__ void load8(const float *p, float (&v)[8]) {
    const float4 a = reinterpret_cast<const float4 *>(p)[0];
    const float4 b = reinterpret_cast<const float4 *>(p)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

template <Prep M>
__global__ __launch_bounds__(256) void prep_batch_kernel(const PrepArgs a) {
    const uint32_t t = blockIdx.x;
    const uint32_t gpr = a.k >> 6;
    const uint32_t tile = t / kTokenTile;
    const uint32_t tt = t % kTokenTile;
    const bool real = t < a.tokens;
    const float *row = a.x + (size_t)(real ? t : 0) * a.k;
    float inv = 1.0f;
    if constexpr (M == Prep::RmsNorm) {
        // Sum of squares of the row: per thread, then across the workgroup
        // in a fixed order.
        float ss = 0.0f;
        for (uint32_t e = threadIdx.x * 8; e < a.k; e += 256 * 8) {
            float v[8];
            load8(row + e, v);
#pragma unroll
            for (int i = 0; i < 8; ++i) ss = __fadd_rn(ss, __fmul_rn(v[i], v[i]));
        }
        ss = dev::wave_sum(ss);
        __shared__ float wsum[4];
        if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = ss;
        __syncthreads();
        ss = ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
        inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)a.k), a.eps)));
    }
    for (uint32_t e = threadIdx.x * 8; e < a.k; e += 256 * 8) {
        float v[8];
        if (real) {
            load8(row + e, v);
            if constexpr (M == Prep::RmsNorm) {
                float w[8];
                load8(a.norm + e, w);
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = __fmul_rn(__fmul_rn(v[i], inv), w[i]);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = 0.0f;
        }
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
        amax = fmaxf(amax, dev::xor_lane<1>(amax));
        amax = fmaxf(amax, dev::xor_lane<2>(amax));
        amax = fmaxf(amax, dev::xor_lane<4>(amax));
        const int ex = dev::chunk_exponent(amax);
        const float up = __builtin_ldexpf(1.0f, 22 - ex);
        uint32_t u[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) u[i] = (uint32_t)((int)__builtin_rintf(v[i] * up) + 0x808080) ^ 0x808080u;
        const uint32_t g = e >> 6;
        const uint32_t j = (e >> 3) & 7u;  // 8-value block within the group
        uint8_t *dst = a.digits + ((size_t)tile * gpr + g) * kGroupBytes + tt * 64 + j * 8;
#pragma unroll
        for (int p = 0; p < 3; ++p) {
            const int sh = 8 * p;
            uint2 w;
            w.x = ((u[0] >> sh) & 0xffu) | (((u[2] >> sh) & 0xffu) << 8) | (((u[4] >> sh) & 0xffu) << 16) |
                  (((u[6] >> sh) & 0xffu) << 24);
            w.y = ((u[1] >> sh) & 0xffu) | (((u[3] >> sh) & 0xffu) << 8) | (((u[5] >> sh) & 0xffu) << 16) |
                  (((u[7] >> sh) & 0xffu) << 24);
            *reinterpret_cast<uint2 *>(dst + p * kPlaneBytes) = w;
        }
        if (j == 0) a.mult[((size_t)tile * gpr + g) * kTokenTile + tt] = __builtin_ldexpf(1.0f, ex - 22);
    }
}

}  // namespace

size_t batch_digit_bytes(uint32_t tokens, uint32_t cols) {
    const size_t tiles = (tokens + kTokenTile - 1) / kTokenTile;
    const size_t groups = cols / 64;
    return tiles * groups * kGroupBytes + tiles * groups * kTokenTile * sizeof(float) + 256;
}

hipError_t launch_prep_batch(hipStream_t s, const GemvInput &in, uint32_t tokens, uint32_t cols, void *digits) {
    const uint32_t tiles = (tokens + kTokenTile - 1) / kTokenTile;
    PrepArgs p{};
    p.x = in.x;
    p.norm = in.norm;
    p.eps = in.eps;
    p.k = cols;
    p.tokens = tokens;
    p.digits = static_cast<uint8_t *>(digits);
    p.mult = reinterpret_cast<float *>(p.digits + (size_t)tiles * (cols / 64) * kGroupBytes);
    const dim3 grid(tiles * kTokenTile);
    switch (in.mode) {
    case GemvInput::F32: prep_batch_kernel<Prep::F32><<<grid, 256, 0, s>>>(p); break;
    case GemvInput::RmsNorm: prep_batch_kernel<Prep::RmsNorm><<<grid, 256, 0, s>>>(p); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gemv_q4_batch(hipStream_t s, const void *digits, const Matrix &w, uint32_t tokens, float *out,
                                const float *residual, bool pairs) {
    if (pairs && (w.rows & 1u)) return hipErrorInvalidValue;
    const uint32_t tiles = (tokens + kTokenTile - 1) / kTokenTile;
    BatchArgs a{};
    a.digits = static_cast<const uint8_t *>(digits);
    a.mult = reinterpret_cast<const float *>(a.digits + (size_t)tiles * (w.cols / 64) * kGroupBytes);
    a.scales = reinterpret_cast<const uint16_t *>(w.scales);
    a.data = w.data;
    a.out = out;
    a.residual = residual;
    a.n = w.rows;
    a.k = w.cols;
    a.tokens = tokens;
    a.pairs = pairs ? 1u : 0u;
    // Tiles per wave: as many as keep about a workgroup per compute unit
    // (each added tile divides the digit-plane reads per weight byte).
    const uint32_t row_tiles = (w.rows + kRowTile - 1) / kRowTile;
    if (row_tiles >= 4u * 256u) {
        gemv_q4_batch_kernel<4><<<dim3((row_tiles + 3) / 4, tiles), 256, 0, s>>>(a);
    } else if (row_tiles >= 2u * 256u) {
        gemv_q4_batch_kernel<2><<<dim3((row_tiles + 1) / 2, tiles), 256, 0, s>>>(a);
    } else {
        gemv_q4_batch_kernel<1><<<dim3(row_tiles, tiles), 256, 0, s>>>(a);
    }
    return hipGetLastError();
}

}  // namespace qwh
