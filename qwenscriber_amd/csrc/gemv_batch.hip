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
// Work split: see gemv_q4_batch_kernel.
#include <cstdlib>

#include "common.h"
#include "device.h"

namespace qwh {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kTokenTile = 16;
constexpr int kRowTile = 16;
constexpr int kPlaneBytes = kTokenTile * 64;           // one digit plane of a group
constexpr int kGroupBytes = 3 * kPlaneBytes;            // three planes

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

// Work split. A workgroup owns TILES 16-row tiles of the output for one
// 16-token tile; its W wavefronts split K into units of GR groups (wave w
// takes units w, w + W, ...), and their partial sums are added in wavefront
// order through LDS (deterministic). A wavefront issues all loads of a unit
// at once -- one memory round trip per unit:
//   weights  TILES x 16 rows x GR x 32 B, as 16-byte pieces, 64/(2 GR) rows
//            per load instruction (each instruction reads whole GR x 32-byte
//            stretches of rows, which streams; 8-byte loads of 16 rows per
//            instruction measured 35 % slower), then moved through this
//            wavefront's LDS into the MFMA operand layout (piece p of row r at
//            slot p ^ (r mod 2 GR): the 16 rows one read touches hit distinct
//            banks);
//   digits   GR x 3 planes x 16 bytes per lane;
//   scales   GR per row (one load per tile), multipliers GR float4s.
template <int TILES, int GR>
struct BatchShape {
    static constexpr int ROWS = kRowTile * TILES;
    static constexpr int PPR = 2 * GR;            // 16-byte pieces of a row in a unit
    static constexpr int RPI = 64 / PPR;          // rows per load instruction
    static constexpr int NW = (ROWS + RPI - 1) / RPI;  // weight loads per lane and unit
    static constexpr int WAVE_BYTES = ROWS * PPR * 16 + TILES * 4 * 64 * 4;  // transpose + partial sums
    static_assert(RPI >= 1 && (ROWS % RPI == 0 || NW == 1), "unit shape");
};

// Wavefronts per workgroup at most: 12 with one tile (up to K = 6144 in one
// unit per wave), 8 otherwise (registers).
template <int TILES>
constexpr int max_waves() { return TILES == 1 ? 12 : 8; }

template <int TILES, int GR>
__global__ __launch_bounds__(64 * max_waves<TILES>()) void gemv_q4_batch_kernel(const BatchArgs a) {
    using S = BatchShape<TILES, GR>;
    constexpr int ROWS = S::ROWS, PPR = S::PPR, RPI = S::RPI, NW = S::NW;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int waves = blockDim.x >> 6;
    const int col = lane & 15;     // weight row within a tile / token within the token tile
    const int blk = lane >> 4;     // 16-column block of the group
    const uint32_t gpr = a.k >> 6;
    const uint32_t units = gpr / GR;
    const uint32_t tile = blockIdx.y;
    const uint32_t row0 = blockIdx.x * ROWS;
    const size_t row_bytes = a.k >> 1;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    uint4 *wl = reinterpret_cast<uint4 *>(smem + (size_t)wave * ROWS * PPR * 16);   // this wave's transpose
    float *part = reinterpret_cast<float *>(smem + (size_t)waves * ROWS * PPR * 16);  // [W][TILES][4][64]

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
    const uint8_t *dig = a.digits + (size_t)tile * gpr * kGroupBytes + col * 64 + blk * 16;
    const float *mul = a.mult + (size_t)tile * gpr * kTokenTile + blk * 4;
    float acc[TILES][4] = {};
    for (uint32_t unit = wave; unit < units; unit += waves) {
        const uint32_t g0 = unit * GR;
        // Loads (rows past the matrix read its last row; their results are
        // never stored).
        uint4 wv[NW];
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            uint32_t row = row0 + i * RPI + lane / PPR;
            if (row >= a.n) row = a.n - 1;
            wv[i] = *reinterpret_cast<const uint4 *>(a.data + (size_t)row * row_bytes + g0 * 32 + 16 * (lane % PPR));
        }
        v4i dg[GR][3];
        float4 mt[GR];
#pragma unroll
        for (int i = 0; i < GR; ++i) {
#pragma unroll
            for (int p = 0; p < 3; ++p)
                dg[i][p] = *reinterpret_cast<const v4i *>(dig + (size_t)(g0 + i) * kGroupBytes + p * kPlaneBytes);
            mt[i] = *reinterpret_cast<const float4 *>(mul + (size_t)(g0 + i) * kTokenTile);
        }
        uint32_t sc[TILES][(GR + 1) / 2];
#pragma unroll
        for (int t = 0; t < TILES; ++t) {
            uint32_t row = row0 + t * kRowTile + col;
            if (row >= a.n) row = a.n - 1;
            __builtin_memcpy(sc[t], a.scales + (size_t)row * gpr + g0, 2 * GR);
        }
        // Weights into the MFMA layout through LDS (this wavefront's region
        // only: LDS operations of one wavefront complete in order).
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            const int r = i * RPI + lane / PPR;
            if (r < ROWS) wl[r * PPR + ((lane % PPR) ^ (r % PPR))] = wv[i];  // (rows past the tile: GR = 1)
        }
#pragma unroll
        for (int i = 0; i < GR; ++i) {
            const float m[4] = {mt[i].x, mt[i].y, mt[i].z, mt[i].w};
#pragma unroll
            for (int t = 0; t < TILES; ++t) {
                const int r = t * kRowTile + col;
                const int piece = 2 * i + (blk >> 1);
                const uint2 w8 = *reinterpret_cast<const uint2 *>(
                    reinterpret_cast<const uint8_t *>(&wl[r * PPR + (piece ^ (r % PPR))]) + 8 * (blk & 1));
                const v4i b = expand_q4(w8);
                const v4i zero = {0, 0, 0, 0};
                const v4i d0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(dg[i][0], b, zero, 0, 0, 0);
                const v4i d1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(dg[i][1], b, zero, 0, 0, 0);
                const v4i d2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(dg[i][2], b, zero, 0, 0, 0);
                const float sv = dev::f16_bits_to_f32((uint16_t)(sc[t][i / 2] >> (16 * (i % 2))));
                const int p0[4] = {d0.x, d0.y, d0.z, d0.w};
                const int p1[4] = {d1.x, d1.y, d1.z, d1.w};
                const int p2[4] = {d2.x, d2.y, d2.z, d2.w};
#pragma unroll
                for (int r2 = 0; r2 < 4; ++r2) {
                    const float f = (float)(p0[r2] + p1[r2] * 256) + 65536.0f * (float)p2[r2];
                    acc[t][r2] = fmaf(f, sv * m[r2], acc[t][r2]);
                }
            }
        }
    }

    // Lane l holds tokens 4 * (l / 16) + r of weight row l % 16 of each tile.
#pragma unroll
    for (int t = 0; t < TILES; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) part[((wave * TILES + t) * 4 + r) * 64 + lane] = acc[t][r];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
        const uint32_t out_row = row0 + t * kRowTile + col;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t tok = tile * kTokenTile + blk * 4 + r;
            float total = part[(t * 4 + r) * 64 + lane];
            for (int w = 1; w < waves; ++w) total += part[((w * TILES + t) * 4 + r) * 64 + lane];
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

// ITERS > 0: K <= 2048 ITERS, and each thread loads all its values (and norm
// weights) at once, keeps them in registers for both passes, so the kernel
// is one memory round trip; ITERS == 0: any K, loaded stretch by stretch.
template <Prep M, int ITERS>
__global__ __launch_bounds__(256) void prep_batch_kernel(const PrepArgs a) {
    const uint32_t t = blockIdx.x;
    const uint32_t gpr = a.k >> 6;
    const uint32_t tile = t / kTokenTile;
    const uint32_t tt = t % kTokenTile;
    const bool real = t < a.tokens;
    const float *row = a.x + (size_t)(real ? t : 0) * a.k;
    constexpr int kHeld = ITERS > 0 ? ITERS : 1;
    float held[kHeld][8], norm_w[kHeld][8];
    if constexpr (ITERS > 0) {
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
            const uint32_t e = threadIdx.x * 8 + 2048u * it;
            const uint32_t ec = e < a.k ? e : 0;  // past the row: a valid address, never used
            load8(row + ec, held[it]);
            if constexpr (M == Prep::RmsNorm) load8(a.norm + ec, norm_w[it]);
        }
    }
    float inv = 1.0f;
    if constexpr (M == Prep::RmsNorm) {
        // Sum of squares of the row: per thread, then across the workgroup
        // in a fixed order.
        float ss = 0.0f;
        if constexpr (ITERS > 0) {
#pragma unroll
            for (int it = 0; it < ITERS; ++it)
                if (threadIdx.x * 8 + 2048u * it < a.k)
#pragma unroll
                    for (int i = 0; i < 8; ++i) ss = __fadd_rn(ss, __fmul_rn(held[it][i], held[it][i]));
        } else {
            for (uint32_t e = threadIdx.x * 8; e < a.k; e += 256 * 8) {
                float v[8];
                load8(row + e, v);
#pragma unroll
                for (int i = 0; i < 8; ++i) ss = __fadd_rn(ss, __fmul_rn(v[i], v[i]));
            }
        }
        ss = dev::wave_sum(ss);
        __shared__ float wsum[4];
        if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = ss;
        __syncthreads();
        ss = ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
        inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)a.k), a.eps)));
    }
    auto encode = [&](uint32_t e, float (&v)[8]) {
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
    };
    if constexpr (ITERS > 0) {
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
            const uint32_t e = threadIdx.x * 8 + 2048u * it;
            if (e >= a.k) break;  // (whole 64-value groups: 8 consecutive threads stop together)
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                float x = real ? held[it][i] : 0.0f;
                if constexpr (M == Prep::RmsNorm) x = __fmul_rn(__fmul_rn(x, inv), norm_w[it][i]);
                v[i] = x;
            }
            encode(e, v);
        }
    } else {
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
            encode(e, v);
        }
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
    const uint32_t iters = (cols + 2047) / 2048;
#define QWH_PREP_CASE(M_)                                                                             \
    switch (iters) {                                                                                  \
    case 1: prep_batch_kernel<M_, 1><<<grid, 256, 0, s>>>(p); break;                                 \
    case 2: prep_batch_kernel<M_, 2><<<grid, 256, 0, s>>>(p); break;                                 \
    case 3: prep_batch_kernel<M_, 3><<<grid, 256, 0, s>>>(p); break;                                 \
    case 4: prep_batch_kernel<M_, 4><<<grid, 256, 0, s>>>(p); break;                                 \
    default: prep_batch_kernel<M_, 0><<<grid, 256, 0, s>>>(p); break;                                \
    }
    switch (in.mode) {
    case GemvInput::F32: QWH_PREP_CASE(Prep::F32) break;
    case GemvInput::RmsNorm: QWH_PREP_CASE(Prep::RmsNorm) break;
    default: return hipErrorInvalidValue;
    }
#undef QWH_PREP_CASE
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
    // Tiles per workgroup: one (measured fastest up to the 12288-row gate|up
    // projection), four for the very tall vocabulary projection (each added
    // tile divides the digit-plane reads per weight byte).
    const uint32_t row_tiles = (w.rows + kRowTile - 1) / kRowTile;
    const uint32_t gpr = w.cols / 64;
    int tiles_per = row_tiles >= 4096u ? 4 : 1;
    if (const char *env = getenv("QWH_BATCH_TILES")) {  // tuning override: 1, 2 or 4
        const int v = atoi(env);
        if (v == 1 || v == 2 || v == 4) tiles_per = v;
    }
    // Groups per unit: 8 (4 with 4 tiles, for registers), lowered to divide
    // the row's groups.
    int gr = tiles_per >= 4 ? 4 : 8;
    while (gpr % (uint32_t)gr) gr >>= 1;
    const uint32_t units = gpr / (uint32_t)gr;
    dim3 grid((row_tiles + tiles_per - 1) / tiles_per, tiles);
#define QWH_BATCH_CASE(T_, G_)                                                                       \
    if (tiles_per == T_ && gr == G_) {                                                               \
        using S = BatchShape<T_, G_>;                                                                \
        /* Wavefronts: the largest divisor of the unit count within the cap and 64 KB of LDS. */     \
        uint32_t waves = 1;                                                                          \
        for (uint32_t c = 1; c <= (uint32_t)max_waves<T_>() && c * S::WAVE_BYTES <= 65536u; ++c)     \
            if (units % c == 0) waves = c;                                                           \
        gemv_q4_batch_kernel<T_, G_><<<grid, 64 * waves, waves * S::WAVE_BYTES, s>>>(a);             \
        return hipGetLastError();                                                                    \
    }
    QWH_BATCH_CASE(1, 8) QWH_BATCH_CASE(1, 4) QWH_BATCH_CASE(1, 2) QWH_BATCH_CASE(1, 1)
    QWH_BATCH_CASE(2, 8) QWH_BATCH_CASE(2, 4) QWH_BATCH_CASE(2, 2) QWH_BATCH_CASE(2, 1)
    QWH_BATCH_CASE(4, 4) QWH_BATCH_CASE(4, 2) QWH_BATCH_CASE(4, 1)
#undef QWH_BATCH_CASE
    return hipErrorInvalidValue;
}

}  // namespace qwh
