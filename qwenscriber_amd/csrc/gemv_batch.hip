// Small-batch q4 / q8 GEMV on the matrix cores: kernels.zig:118-158
// linearQuantized for 2 or more tokens (the decoder step at batch > 1).
//
// One v_mfma_i32_16x16x64_i8 multiplies 16 tokens by 16 weight rows over 64
// consecutive columns -- exactly one quantization group (quant.zig:49), so
// its integer result takes that group's single f16 scale per row. The
// operands are exact integers:
//   weights      the codes u - 8 (q4) or u - 128 (q8) as signed bytes;
//   activations  per token and group, x_int = rint(x * 2^(22-e)) with 2^e
//                bounding the group's largest |x| (|x_int| <= 2^22), written
//                as three signed base-256 digit planes d0 + 256 d1 + 65536 d2
//                (d in [-128, 127]); one MFMA per plane.
// Each plane's dot product is below 2^16 in magnitude, so the int32 results
// are exact; they are combined in f32 and scaled by f16 scale * 2^(e-22).
//
// Operand layout. Lane l of a wavefront feeds token (or weight row) l % 16
// and the 16 columns 16 * (l / 16) .. +15 of the group. A lane's 16 codes are
// 8 bytes of a q4 row (two per byte, even column in the low nibble,
// quant.zig:36-41), which nibble masks split into the bytes of columns
// {0,2,4,6}, {1,3,5,7}, {8,10,12,14}, {9,11,13,15}; or 16 bytes of a q8 row,
// which v_perm_b32 puts in that same order. The activation digits are stored
// in that order too, so byte b of both operands belongs to the same column. Layout of the digits, per 16-token tile and group:
//   digits[tile][g][plane][token 0..15][64 bytes],  mult[tile][g][16] f32.
//
// Work split: see gemv_batch_kernel.
#include <algorithm>
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

// The same operand from 16 q8 codes (columns 0..15 in order): the even and
// odd columns of each 8-column block picked by v_perm_b32, XOR 0x80 making
// each byte the two's complement of u - 128.
__device__ __forceinline__ v4i expand_q8(v4i n) {
    v4i b;
    b.x = (int)(__builtin_amdgcn_perm((uint32_t)n.y, (uint32_t)n.x, 0x06040200u) ^ 0x80808080u);
    b.y = (int)(__builtin_amdgcn_perm((uint32_t)n.y, (uint32_t)n.x, 0x07050301u) ^ 0x80808080u);
    b.z = (int)(__builtin_amdgcn_perm((uint32_t)n.w, (uint32_t)n.z, 0x06040200u) ^ 0x80808080u);
    b.w = (int)(__builtin_amdgcn_perm((uint32_t)n.w, (uint32_t)n.z, 0x07050301u) ^ 0x80808080u);
    return b;
}

// The same operand from a q5 slice of 16 codes (quant.zig:253-269): 8 bytes
// of nibbles (column 2j in the low nibble of byte j) and the slice's 16 fifth
// bits (bit j for column j). The fifth bits of the columns {0,2,4,6} (or
// {1,3,5,7}) of an 8-column block sit at bits 0, 2, 4, 6 of one byte and move
// to bit 4 of bytes 0..3 with one multiply (no carry reaches those bits);
// u = nibble | fifth << 4 in [0, 31], and (u + 0x70) ^ 0x80 is u - 16 as a
// two's complement byte.
__device__ __forceinline__ uint32_t spread_fifths(uint32_t b) { return ((b & 0x55u) * 0x00410410u) & 0x10101010u; }

__device__ __forceinline__ v4i expand_q5(uint2 nib, uint32_t fifth) {
    const uint32_t fe = fifth & 0x5555u, fo = (fifth >> 1) & 0x5555u;
    v4i b;
    b.x = (int)((((nib.x & 0x0f0f0f0fu) | spread_fifths(fe)) + 0x70707070u) ^ 0x80808080u);
    b.y = (int)(((((nib.x >> 4) & 0x0f0f0f0fu) | spread_fifths(fo)) + 0x70707070u) ^ 0x80808080u);
    b.z = (int)((((nib.y & 0x0f0f0f0fu) | spread_fifths(fe >> 8)) + 0x70707070u) ^ 0x80808080u);
    b.w = (int)(((((nib.y >> 4) & 0x0f0f0f0fu) | spread_fifths(fo >> 8)) + 0x70707070u) ^ 0x80808080u);
    return b;
}

// The weight operand of group i, rows r of a wavefront's LDS transpose
// (PPR 16-byte pieces per row, piece p of row r at slot p ^ (r mod PPR)):
// BPG = 32 (q4) or 64 (q8) code bytes per group.
template <int BPG, int PPR>
__device__ __forceinline__ v4i weight_operand(const v4i *wl, int r, int i, int blk) {
    if constexpr (BPG == 32) {
        const int piece = 2 * i + (blk >> 1);
        const uint2 w8 = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint8_t *>(&wl[r * PPR + (piece ^ (r % PPR))]) +
                                                          8 * (blk & 1));
        return expand_q4(w8);
    } else {
        const int piece = 4 * i + blk;
        return expand_q8(wl[r * PPR + (piece ^ (r % PPR))]);
    }
}

struct BatchArgs {
    const uint8_t *digits;   // [token tiles][groups][3][16][64]
    const float *mult;       // [token tiles][groups][16]
    const uint16_t *scales;  // N * K/64
    const uint8_t *data;     // N * K/64 * BPG
    float *out;              // tokens x N, or tokens x N/2 with pairs
    const float *residual;   // optional, tokens x N (may alias out); not with pairs
    const float *bias;       // optional, N: out = residual + (W x + bias); not with pairs
    const float *ss;         // non-null: RMSNorm sums of squares [token][ss_parts]; results x 1/rms
    uint32_t ss_parts;
    float eps;
    uint32_t n, k, tokens;
    uint32_t pairs;          // rows 2j, 2j+1 are gate_j, up_j: write silu(gate_j) * up_j
};

// siluMul of one gate / up pair (math.zig:69-71: silu(g) = g / (1 + exp(-g))).
__device__ __forceinline__ float silu_mul(float g, float u) {
    return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, expf(-g))), u);
}

// 1 / sqrt(ss / K + eps) (math.zig:120-130), from the sums of squares the
// prep left per 512-value stretch, added in stretch order.
__device__ __forceinline__ float rms_inverse(const float *parts, uint32_t n, uint32_t k, float eps) {
    float ss = 0.0f;
    for (uint32_t p = 0; p < n; ++p) ss = __fadd_rn(ss, parts[p]);
    return __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)k), eps)));
}

// The factor of token 4 (lane / 16) + r for each r, with lane t < 16 of the
// wavefront computing token t's once (`parts` = [token][n] for the 16-token
// tile; a tile with tokens past the batch reads their zero sums).
__device__ __forceinline__ void tile_rms_inverse(const float *parts, uint32_t n, uint32_t k, float eps, int lane,
                                                 float (&inv)[4]) {
    float mine = 1.0f;
    if (lane < 16) mine = rms_inverse(parts + lane * n, n, k, eps);
#pragma unroll
    for (int r = 0; r < 4; ++r) inv[r] = __shfl(mine, (lane >> 4) * 4 + r, 64);
}

// Work split. A workgroup owns TILES 16-row tiles of the output for one
// 16-token tile; its W wavefronts split K into units of GR groups (wave w
// takes units w, w + W, ...), and their partial sums are added in wavefront
// order through LDS (deterministic). A wavefront issues all loads of a unit
// at once -- one memory round trip per unit:
//   weights  TILES x 16 rows x GR x BPG B, as 16-byte pieces, 64/PPR rows
//            per load instruction (each instruction reads whole GR x 32-byte
//            stretches of rows, which streams; 8-byte loads of 16 rows per
//            instruction measured 35 % slower), then moved through this
//            wavefront's LDS into the MFMA operand layout (piece p of row r at
//            slot p ^ (r mod 2 GR): the 16 rows one read touches hit distinct
//            banks);
//   digits   GR x 3 planes x 16 bytes per lane;
//   scales   GR per row (one load per tile), multipliers GR float4s.
template <int TILES, int GR, int BPG>
struct BatchShape {
    static constexpr int ROWS = kRowTile * TILES;
    static constexpr int PPR = BPG * GR / 16;     // 16-byte pieces of a row in a unit
    static constexpr int RPI = 64 / PPR;          // rows per load instruction
    static constexpr int NW = (ROWS + RPI - 1) / RPI;  // weight loads per lane and unit
    static constexpr int WAVE_BYTES = ROWS * PPR * 16 + TILES * 4 * 64 * 4;  // transpose + partial sums
    static_assert(RPI >= 1 && (ROWS % RPI == 0 || NW == 1), "unit shape");
};

// Wavefronts per workgroup at most: 12 with one tile (up to K = 6144 in one
// unit per wave), 8 otherwise (registers).
template <int TILES>
constexpr int max_waves() { return TILES == 1 ? 12 : 8; }

template <int TILES, int GR, int BPG>
__global__ __launch_bounds__(64 * max_waves<TILES>()) void gemv_batch_kernel(const BatchArgs a) {
    using S = BatchShape<TILES, GR, BPG>;
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
    const size_t row_bytes = (size_t)gpr * BPG;
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
            wv[i] = *reinterpret_cast<const uint4 *>(a.data + (size_t)row * row_bytes + g0 * BPG + 16 * (lane % PPR));
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
                const v4i b = weight_operand<BPG, PPR>(reinterpret_cast<const v4i *>(wl), r, i, blk);
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
    float inv[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    if (a.ss) tile_rms_inverse(a.ss + (size_t)tile * kTokenTile * a.ss_parts, a.ss_parts, a.k, a.eps, lane, inv);
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
        const uint32_t out_row = row0 + t * kRowTile + col;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t tok = tile * kTokenTile + blk * 4 + r;
            float total = part[(t * 4 + r) * 64 + lane];
            for (int w = 1; w < waves; ++w) total += part[((w * TILES + t) * 4 + r) * 64 + lane];
            if (a.ss) total = __fmul_rn(total, inv[r]);
            if (a.pairs) {
                // Row + 1 is the next lane's row (same token).
                const float partner = __shfl_down(total, 1, 64);
                if (tok < a.tokens && (out_row & 1u) == 0 && out_row < a.n)
                    a.out[(size_t)tok * (a.n / 2) + (out_row >> 1)] = silu_mul(total, partner);
            } else if (tok < a.tokens && out_row < a.n) {
                a.out[(size_t)tok * a.n + out_row] = res[t][r] + (a.bias ? total + a.bias[out_row] : total);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Split form. Every workgroup of the form above reads all of K's digit
// planes (48 B per column for a 16-token tile), several times the weight
// bytes of its few rows, and those reads set its time. Here a workgroup of
// four wavefronts covers 4 x 16 TW rows (wavefront w: TW tiles from
// 16 TW w) and one K slice; the slice is walked in chunks of KC groups whose
// digit planes are read once per workgroup and staged in LDS for all four
// wavefronts (in lane order: conflict-free 16-byte reads), while the next
// chunk's weights, digits, multipliers and scales are already in flight.
// Weights move into the MFMA layout through each wavefront's own LDS region
// as above. The workgroup writes either the output (+ residual, silu pairs;
// one slice only) or its slice's partial sums to part[slice][token][row],
// which the next kernel adds in slice order: split_reduce_kernel, or the
// batch prep that consumes them (the residual stream, silu pairs).
// ---------------------------------------------------------------------------
constexpr uint32_t kMaxSlices = 8;

struct SplitArgs {
    const uint8_t *digits;
    const float *mult;
    const uint16_t *scales;
    const uint8_t *data;
    float *out;
    const float *residual;
    const float *bias;       // optional, n: out = residual + (W x + bias) (one slice, no pairs)
    float *part;             // non-null: partial sums [slices][tokens][n] instead of out
    const float *ss;         // non-null: RMSNorm sums of squares [token][ss_parts]; results x 1/rms
    uint32_t ss_parts;
    float eps;
    uint32_t n, k, tokens;
    uint32_t pairs;
    uint32_t slice_groups;   // groups per K slice (a multiple of KC)
};


template <int TW, int KC, int BPG>
struct SplitShape {
    static constexpr int ROWS = kRowTile * TW;      // rows per wavefront
    static constexpr int PPR = BPG * KC / 16;       // 16-byte pieces of a row in a chunk
    static constexpr int RPI = 64 / PPR;            // rows per load instruction
    static constexpr int NW = (ROWS + RPI - 1) / RPI;
    static constexpr int DPIECES = KC * 3 * 64;     // 16-byte digit pieces per chunk
    static constexpr int DPT = (DPIECES + 255) / 256;  // ... per thread (the last round partly idle)
    static_assert(DPIECES % 128 == 0 && (PPR & (PPR - 1)) == 0 && ROWS % RPI == 0, "chunk shape");
};

// The end of a split GEMV workgroup: lane l holds tokens 4 (l / 16) + r of
// row l % 16 of each of its TW tiles; it writes its K slice's partial sums,
// or (one slice) the outputs plus residual, or silu pairs.
template <int TW>
__device__ __forceinline__ void split_epilogue(const SplitArgs &a, const float (&acc)[TW][4], uint32_t tile,
                                               uint32_t row0, int col, int blk) {
    if (a.part) {
#pragma unroll
        for (int t = 0; t < TW; ++t) {
            const uint32_t out_row = row0 + t * kRowTile + col;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t tok = tile * kTokenTile + blk * 4 + r;
                if (tok < a.tokens && out_row < a.n)
                    a.part[((size_t)blockIdx.y * a.tokens + tok) * a.n + out_row] = acc[t][r];
            }
        }
        return;
    }
#pragma unroll
    for (int t = 0; t < TW; ++t) {
        const uint32_t out_row = row0 + t * kRowTile + col;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t tok = tile * kTokenTile + blk * 4 + r;
            const float total = acc[t][r];
            if (a.pairs) {
                const float partner = __shfl_down(total, 1, 64);
                if (tok < a.tokens && (out_row & 1u) == 0 && out_row < a.n)
                    a.out[(size_t)tok * (a.n / 2) + (out_row >> 1)] = silu_mul(total, partner);
            } else if (tok < a.tokens && out_row < a.n) {
                const float res = a.residual ? a.residual[(size_t)tok * a.n + out_row] : 0.0f;
                a.out[(size_t)tok * a.n + out_row] = res + (a.bias ? total + a.bias[out_row] : total);
            }
        }
    }
}

// The split workgroup for row block `bx` of `a`'s matrix.
template <int TW, int KC, int BPG>
__device__ __forceinline__ void split_block(const SplitArgs &a, uint32_t bx) {
    using S = SplitShape<TW, KC, BPG>;
    constexpr int ROWS = S::ROWS, PPR = S::PPR, RPI = S::RPI, NW = S::NW, DPT = S::DPT;
    __shared__ v4i dl[2][S::DPIECES];          // digit planes, [group][plane][lane]
    __shared__ float4 ml[2][KC * 4];             // multipliers, [group][lane / 16]
    __shared__ v4i wls[4][ROWS * PPR];         // per-wavefront weight transpose
    __shared__ float ssl[kTokenTile * 16];       // RMSNorm sums of squares of the token tile
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int col = lane & 15;
    const int blk = lane >> 4;
    const uint32_t gpr = a.k >> 6;
    const uint32_t tile = blockIdx.z;
    const uint32_t row0 = (bx * 4 + wave) * ROWS;
    const size_t row_bytes = (size_t)gpr * BPG;
    const uint32_t g_first = blockIdx.y * a.slice_groups;
    const uint32_t chunks = a.slice_groups / KC;
    const uint8_t *dig = a.digits + (size_t)tile * gpr * kGroupBytes;
    const float *mul = a.mult + (size_t)tile * gpr * kTokenTile;
    v4i *wl = wls[wave];

    // (Native vector types: these stay in registers across the chunk loop.)
    v4i rw[NW], rd[DPT];
    float4 rm = {};
    uint32_t rs[TW][KC / 2];
    // One chunk's loads (rows past the matrix read its last row; their
    // results are never stored).
    auto load = [&](uint32_t g0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            uint32_t row = row0 + i * RPI + lane / PPR;
            if (row >= a.n) row = a.n - 1;
            rw[i] = *reinterpret_cast<const v4i *>(a.data + (size_t)row * row_bytes + g0 * BPG + 16 * (lane % PPR));
        }
#pragma unroll
        for (int m = 0; m < DPT; ++m) {
            // Piece q = (group, plane, lane L) of lane order; lane L reads
            // column block L / 16 of token L % 16. (Threads past the
            // chunk's pieces load the last one again and do not store it:
            // the load stays unconditional.)
            const int q = tid + 256 * m < S::DPIECES ? tid + 256 * m : S::DPIECES - 1;
            const int L = q & 63;
            rd[m] = *reinterpret_cast<const v4i *>(dig + ((size_t)g0 * 3 + (q >> 6)) * kPlaneBytes +
                                                     (L & 15) * 64 + (L >> 4) * 16);
        }
        // (Every thread loads, the first KC * 4 their own float4: a load
        // under a branch would make the wait counts conservative.)
        rm = *reinterpret_cast<const float4 *>(mul + (size_t)g0 * kTokenTile + (tid % (KC * 4)) * 4);
#pragma unroll
        for (int t = 0; t < TW; ++t) {
            uint32_t row = row0 + t * kRowTile + col;
            if (row >= a.n) row = a.n - 1;
            __builtin_memcpy(rs[t], a.scales + (size_t)row * gpr + g0, 2 * KC);
        }
    };

    float acc[TW][4] = {};
    float inv[4] = {1.0f, 1.0f, 1.0f, 1.0f};  // 1 / rms of the lane's tokens (RMSNorm input)
    // The token tile's sums of squares travel with the first chunk.
    const bool has_ss = a.ss && (uint32_t)tid < kTokenTile * a.ss_parts;
    const float ssv = has_ss ? a.ss[(size_t)tile * kTokenTile * a.ss_parts + tid] : 0.0f;
    load(g_first);
    for (uint32_t c = 0; c < chunks; ++c) {
        const int buf = c & 1;
        if (c == 0 && has_ss) ssl[tid] = ssv;
#pragma unroll
        for (int m = 0; m < DPT; ++m)
            if (tid + 256 * m < S::DPIECES) dl[buf][tid + 256 * m] = rd[m];
        if (tid < KC * 4) ml[buf][tid] = rm;
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            const int r = i * RPI + lane / PPR;
            wl[r * PPR + ((lane % PPR) ^ (r % PPR))] = rw[i];
        }
        float sc[TW][KC];  // this chunk's scales, converted before the next chunk's loads go out
#pragma unroll
        for (int t = 0; t < TW; ++t)
#pragma unroll
            for (int i = 0; i < KC; ++i) sc[t][i] = dev::f16_bits_to_f32((uint16_t)(rs[t][i / 2] >> (16 * (i % 2))));
        // The other wavefronts' digits are in; the buffer written next
        // iteration was last read before this barrier.
        __syncthreads();
        // The next chunk's loads (the last iteration reloads its own chunk:
        // an unconditional load keeps them in flight across the products).
        load(g_first + (c + 1 < chunks ? c + 1 : c) * KC);
        if (c == 0 && a.ss) tile_rms_inverse(ssl, a.ss_parts, a.k, a.eps, lane, inv);  // (beside the products)
#pragma unroll
        for (int i = 0; i < KC; ++i) {
            const v4i d0 = dl[buf][(i * 3 + 0) * 64 + lane];
            const v4i d1 = dl[buf][(i * 3 + 1) * 64 + lane];
            const v4i d2 = dl[buf][(i * 3 + 2) * 64 + lane];
            const float4 mm = ml[buf][i * 4 + blk];
            const float m[4] = {mm.x, mm.y, mm.z, mm.w};
#pragma unroll
            for (int t = 0; t < TW; ++t) {
                const int r = t * kRowTile + col;
                const v4i b = weight_operand<BPG, PPR>(wl, r, i, blk);
                const v4i zero = {0, 0, 0, 0};
                const v4i p0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(d0, b, zero, 0, 0, 0);
                const v4i p1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(d1, b, zero, 0, 0, 0);
                const v4i p2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(d2, b, zero, 0, 0, 0);
                const float sv = sc[t][i];
                const int q0[4] = {p0.x, p0.y, p0.z, p0.w};
                const int q1[4] = {p1.x, p1.y, p1.z, p1.w};
                const int q2[4] = {p2.x, p2.y, p2.z, p2.w};
#pragma unroll
                for (int r2 = 0; r2 < 4; ++r2) {
                    const float f = (float)(q0[r2] + q1[r2] * 256) + 65536.0f * (float)q2[r2];
                    acc[t][r2] = fmaf(f, sv * m[r2], acc[t][r2]);
                }
            }
        }
    }

    // Lane l holds tokens 4 (l / 16) + r of row l % 16 of each tile.
    if (a.ss)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int t = 0; t < TW; ++t) acc[t][r] = __fmul_rn(acc[t][r], inv[r]);
    split_epilogue<TW>(a, acc, tile, row0, col, blk);
}

template <int TW, int KC, int BPG>
__global__ __launch_bounds__(256) void gemv_split_kernel(const SplitArgs a) {
    split_block<TW, KC, BPG>(a, blockIdx.x);
}

// Up to three matrices of one shape class (format, K, plan; one K slice)
// over the same activation digits in one launch: grid.x runs over the
// matrices' row blocks in order.
constexpr int kMaxMulti = 3;
struct SplitMulti {
    SplitArgs m[kMaxMulti];
    uint32_t blocks[kMaxMulti];
    uint32_t count;
};

template <int TW, int KC, int BPG>
__global__ __launch_bounds__(256) void gemv_split_multi_kernel(const SplitMulti s) {
    uint32_t bx = blockIdx.x, i = 0;
    while (i + 1 < s.count && bx >= s.blocks[i]) bx -= s.blocks[i++];
    split_block<TW, KC, BPG>(s.m[i], bx);
}

// Sum over the K slices, in slice order, of the partial sums at p (slices
// planes `plane` floats apart). All loads are issued before the first add.
__device__ __forceinline__ float slice_sum(const float *p, uint32_t slices, size_t plane) {
    float w[kMaxSlices];
#pragma unroll
    for (uint32_t s = 0; s < kMaxSlices; ++s)
        if (s < slices) w[s] = p[s * plane];
    float v = w[0];
#pragma unroll
    for (uint32_t s = 1; s < kMaxSlices; ++s)
        if (s < slices) v += w[s];
    return v;
}

__device__ __forceinline__ float4 slice_sum4(const float *p, uint32_t slices, size_t plane) {
    float4 w[kMaxSlices];
#pragma unroll
    for (uint32_t s = 0; s < kMaxSlices; ++s)
        if (s < slices) w[s] = *reinterpret_cast<const float4 *>(p + s * plane);
    float4 v = w[0];
#pragma unroll
    for (uint32_t s = 1; s < kMaxSlices; ++s)
        if (s < slices) {
            v.x += w[s].x;
            v.y += w[s].y;
            v.z += w[s].z;
            v.w += w[s].w;
        }
    return v;
}

// The split form over q5 codes. A 40-byte group does not cut into the
// 16-byte pieces of the LDS weight transpose, so each lane loads its own
// operand bytes (the 8 nibble bytes and 2 fifth-bit bytes of its 16 columns,
// for each of its tiles and the chunk's groups) straight into registers, one
// chunk ahead; the digits, multipliers, scales, split and epilogue are those
// of gemv_split_kernel, with chunks of KC = 4 groups, or 2 for rows whose
// group count is not a multiple of 4 (the 0.6B audio tower's 896-wide rows:
// 14 groups).
template <int TW, int KC>
__global__ __launch_bounds__(256) void gemv_split_q5_kernel(const SplitArgs a) {
    using S = SplitShape<TW, KC, 32>;  // (digit staging only)
    constexpr int ROWS = S::ROWS, DPT = S::DPT;
    // The wavefront's rows of a chunk (KC 40-byte groups each) are loaded as
    // whole 16-byte pieces, consecutive lanes on consecutive pieces, and
    // passed through its own LDS rows (stride RS pieces: the 16 rows one
    // operand read touches fall on distinct banks), from which each lane
    // reads its 8 nibble bytes and 2 fifth-bit bytes per group.
    constexpr int PPR = KC * 40 / 16;          // pieces of a row's chunk
    constexpr int RS = KC == 4 ? 11 : 7;       // LDS row stride, pieces
    constexpr int NP = ROWS * PPR;             // pieces per wavefront and chunk
    constexpr int NWQ = (NP + 63) / 64;        // loads per lane
    static_assert(KC * 40 % 16 == 0 && RS >= PPR, "whole pieces per row");
    __shared__ v4i dl[2][S::DPIECES];
    __shared__ float4 ml[2][KC * 4];
    __shared__ float ssl[kTokenTile * 16];
    __shared__ v4i wq[4][ROWS * RS];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int col = lane & 15;
    const int blk = lane >> 4;
    const uint32_t gpr = a.k >> 6;
    const uint32_t tile = blockIdx.z;
    const uint32_t row0 = (blockIdx.x * 4 + wave) * ROWS;
    const size_t row_bytes = (size_t)gpr * 40;
    const uint32_t g_first = blockIdx.y * a.slice_groups;
    const uint32_t chunks = a.slice_groups / KC;
    const uint8_t *dig = a.digits + (size_t)tile * gpr * kGroupBytes;
    const float *mul = a.mult + (size_t)tile * gpr * kTokenTile;
    v4i *wl = wq[wave];

    v4i rw[NWQ];
    v4i rd[DPT];
    float4 rm = {};
    uint32_t rs[TW][KC / 2];
    // One chunk's loads (rows past the matrix read its last row, pieces
    // past the wavefront's the last piece again; neither is stored).
    auto load = [&](uint32_t g0) __attribute__((always_inline)) {
#pragma unroll
        for (int m = 0; m < NWQ; ++m) {
            const int q = lane + 64 * m < NP ? lane + 64 * m : NP - 1;
            uint32_t row = row0 + q / PPR;
            if (row >= a.n) row = a.n - 1;
            rw[m] = *reinterpret_cast<const v4i *>(a.data + row * row_bytes + (size_t)g0 * 40 + 16 * (q % PPR));
        }
#pragma unroll
        for (int t = 0; t < TW; ++t) {
            uint32_t row = row0 + t * kRowTile + col;
            if (row >= a.n) row = a.n - 1;
            __builtin_memcpy(rs[t], a.scales + (size_t)row * gpr + g0, 2 * KC);
        }
#pragma unroll
        for (int m = 0; m < DPT; ++m) {
            // (Threads past the chunk's pieces load the last one again and
            // do not store it: the load stays unconditional.)
            const int q = tid + 256 * m < S::DPIECES ? tid + 256 * m : S::DPIECES - 1;
            const int L = q & 63;
            rd[m] = *reinterpret_cast<const v4i *>(dig + ((size_t)g0 * 3 + (q >> 6)) * kPlaneBytes +
                                                     (L & 15) * 64 + (L >> 4) * 16);
        }
        rm = *reinterpret_cast<const float4 *>(mul + (size_t)g0 * kTokenTile + (tid % (KC * 4)) * 4);
    };

    float acc[TW][4] = {};
    float inv[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    const bool has_ss = a.ss && (uint32_t)tid < kTokenTile * a.ss_parts;
    const float ssv = has_ss ? a.ss[(size_t)tile * kTokenTile * a.ss_parts + tid] : 0.0f;
    load(g_first);
    for (uint32_t c = 0; c < chunks; ++c) {
        const int buf = c & 1;
        if (c == 0 && has_ss) ssl[tid] = ssv;
#pragma unroll
        for (int m = 0; m < DPT; ++m)
            if (tid + 256 * m < S::DPIECES) dl[buf][tid + 256 * m] = rd[m];
        if (tid < KC * 4) ml[buf][tid] = rm;
#pragma unroll
        for (int m = 0; m < NWQ; ++m) {
            const int q = lane + 64 * m;
            if (q < NP) wl[(q / PPR) * RS + q % PPR] = rw[m];
        }
        // This chunk's operands and scales, out of the registers and LDS
        // rows the next chunk's loads are about to fill.
        v4i wop[TW][KC];
        float sc[TW][KC];
#pragma unroll
        for (int t = 0; t < TW; ++t)
#pragma unroll
            for (int i = 0; i < KC; ++i) {
                const uint8_t *grp = reinterpret_cast<const uint8_t *>(wl + (t * kRowTile + col) * RS) + i * 40;
                wop[t][i] = expand_q5(*reinterpret_cast<const uint2 *>(grp + 8 * blk),
                                      *reinterpret_cast<const uint16_t *>(grp + 32 + 2 * blk));
                sc[t][i] = dev::f16_bits_to_f32((uint16_t)(rs[t][i / 2] >> (16 * (i % 2))));
            }
        __syncthreads();
        load(g_first + (c + 1 < chunks ? c + 1 : c) * KC);
        if (c == 0 && a.ss) tile_rms_inverse(ssl, a.ss_parts, a.k, a.eps, lane, inv);
#pragma unroll
        for (int i = 0; i < KC; ++i) {
            const v4i d0 = dl[buf][(i * 3 + 0) * 64 + lane];
            const v4i d1 = dl[buf][(i * 3 + 1) * 64 + lane];
            const v4i d2 = dl[buf][(i * 3 + 2) * 64 + lane];
            const float4 mm = ml[buf][i * 4 + blk];
            const float m[4] = {mm.x, mm.y, mm.z, mm.w};
#pragma unroll
            for (int t = 0; t < TW; ++t) {
                const v4i zero = {0, 0, 0, 0};
                const v4i p0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(d0, wop[t][i], zero, 0, 0, 0);
                const v4i p1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(d1, wop[t][i], zero, 0, 0, 0);
                const v4i p2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(d2, wop[t][i], zero, 0, 0, 0);
                const int q0[4] = {p0.x, p0.y, p0.z, p0.w};
                const int q1[4] = {p1.x, p1.y, p1.z, p1.w};
                const int q2[4] = {p2.x, p2.y, p2.z, p2.w};
#pragma unroll
                for (int r2 = 0; r2 < 4; ++r2) {
                    const float f = (float)(q0[r2] + q1[r2] * 256) + 65536.0f * (float)q2[r2];
                    acc[t][r2] = fmaf(f, sc[t][i] * m[r2], acc[t][r2]);
                }
            }
        }
    }
    if (a.ss)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int t = 0; t < TW; ++t) acc[t][r] = __fmul_rn(acc[t][r], inv[r]);
    split_epilogue<TW>(a, acc, tile, row0, col, blk);
}

// out = residual + the slice sum (pairs: silu(sum of row 2j) * sum of row
// 2j + 1), one output per thread.
__global__ __launch_bounds__(256) void split_reduce_kernel(const float *part, uint32_t slices, uint32_t tokens,
                                                           uint32_t n, const float *residual, float *out,
                                                           uint32_t pairs, const float *bias) {
    const uint32_t width = pairs ? n / 2 : n;
    const size_t plane = (size_t)tokens * n;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)tokens * width) return;
    const size_t tok = i / width, j = i % width;
    if (pairs) {
        const size_t at = tok * n + 2 * j;
        out[i] = silu_mul(slice_sum(part + at, slices, plane), slice_sum(part + at + 1, slices, plane));
    } else {
        const size_t at = tok * n + j;
        float v = slice_sum(part + at, slices, plane);
        if (bias) v += bias[j];
        out[i] = residual ? residual[at] + v : v;
    }
}

// ---------------------------------------------------------------------------
// Activation digits. One wavefront per 512 values of a token (padding tokens
// of the last tile write zeros): lane i takes values 8i .. 8i+7, so the 8
// lanes of a 64-value group are consecutive. Forms: f32 values as they are;
// RMSNorm (math.zig:120-130) of x, of which this kernel applies only the
// weights -- it encodes x_k * w_k and leaves each wavefront's sum of squares
// of x, and the GEMV multiplies its dot products by the token's
// 1 / sqrt(sum / K + eps) (a per-token factor of a linear map), so no
// wavefront waits for the rest of the row; and with the partial sums of a
// split GEMV folded in: RMSNorm of x + their sum (the residual stream,
// written back), or siluMul of the gate / up sums (math.zig:69-71).
// ---------------------------------------------------------------------------
enum class Prep : int { F32 = 0, RmsNorm = 1, Pairs = 2, BiasGelu = 3 };

constexpr uint32_t kPrepValues = 512;  // values per wavefront

struct PrepArgs {
    const float *x;      // tokens x K (F32, RmsNorm)
    const float *norm;   // RmsNorm weights
    uint32_t k, tokens;
    // Partial sums [slices][tokens][part_n] of the GEMV that produced the
    // input (slices 0: none). RmsNorm: x + their sum, also stored to x_out
    // (may be x); Pairs (part_n = 2K): value j = silu(sum of row 2j) * sum of
    // row 2j + 1.
    const float *part;
    uint32_t slices, part_n;
    float *x_out;
    uint8_t *digits;
    float *mult;
    float *ss;           // RmsNorm: [token][K / 512] sums of squares
    const float *bias;   // BiasGelu: per-column bias added before the GELU
};

__device__ __forceinline__ void load8(const float *p, float (&v)[8]) {
    const float4 a = reinterpret_cast<const float4 *>(p)[0];
    const float4 b = reinterpret_cast<const float4 *>(p)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

__device__ __forceinline__ void store8(float *p, const float (&v)[8]) {
    reinterpret_cast<float4 *>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4 *>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
}

// Input values e .. e + 7 of token t.
template <Prep M>
__device__ __forceinline__ void input8(const PrepArgs &a, uint32_t t, uint32_t e, float (&v)[8]) {
    const size_t plane = (size_t)a.tokens * a.part_n;
    if constexpr (M == Prep::Pairs) {
        const float *p = a.part + (size_t)t * a.part_n + 2 * e;
        float f[16];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float4 q = slice_sum4(p + 4 * j, a.slices, plane);
            f[4 * j] = q.x; f[4 * j + 1] = q.y; f[4 * j + 2] = q.z; f[4 * j + 3] = q.w;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = silu_mul(f[2 * i], f[2 * i + 1]);
    } else {
        load8(a.x + (size_t)t * a.k + e, v);
        if constexpr (M == Prep::BiasGelu) {
            float b[8];
            load8(a.bias + e, b);
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = dev::gelu(v[i] + b[i]);
        }
        if (M == Prep::RmsNorm && a.slices) {
            const float *p = a.part + (size_t)t * a.part_n + e;
            const float4 s0 = slice_sum4(p, a.slices, plane);
            const float4 s1 = slice_sum4(p + 4, a.slices, plane);
            const float sum[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = __fadd_rn(v[i], sum[i]);
        }
    }
}

// Activation digits of values e .. e + 7 (e a multiple of 8) of token tt of
// a 16-token tile: per 64-value group (8 consecutive lanes, which must all
// run this) x_int = rint(x * 2^(22-e)) with 2^e bounding the group's largest
// |x|, three signed base-256 digit planes; within each 8-value block the even
// columns' bytes come first, then the odd ones'. The group's multiplier
// 2^(e-22) is written by its first lane.
__device__ __forceinline__ void encode_digits8(const float (&v)[8], uint32_t tile, uint32_t tt, uint32_t e,
                                               uint32_t gpr, uint8_t *digits, float *mult) {
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
    uint8_t *dst = digits + ((size_t)tile * gpr + g) * kGroupBytes + tt * 64 + j * 8;
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
    if (j == 0) mult[((size_t)tile * gpr + g) * kTokenTile + tt] = __builtin_ldexpf(1.0f, ex - 22);
}

// math.zig:99-116 layerNorm of each token row (one 256-thread workgroup per
// token, the statistics of layer_norm_kernel) written straight as the batch
// GEMV's activation digits (padding tokens of the last tile write zeros).
__global__ __launch_bounds__(256) void layer_norm_digits_kernel(const float *x, const float *weight,
                                                                const float *bias, uint32_t width, uint32_t tokens,
                                                                float eps, uint8_t *digits, float *mult) {
    __shared__ float lds[4];
    const uint32_t t = blockIdx.x;
    const bool real = t < tokens;
    const float *row = x + (size_t)(real ? t : 0) * width;
    float mean, inverse_std;
    dev::layer_norm_stats(row, width, eps, lds, mean, inverse_std);
    const uint32_t gpr = width >> 6;
    for (uint32_t base = 0; base < width; base += 8 * 256) {
        const uint32_t e = base + 8 * threadIdx.x;
        const bool in_row = e < width;  // (whole groups: width is a multiple of 64)
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t c = in_row ? e + i : 0;
            v[i] = real && in_row ? (row[c] - mean) * inverse_std * weight[c] + bias[c] : 0.0f;
        }
        if (in_row) encode_digits8(v, t / kTokenTile, t % kTokenTile, e, gpr, digits, mult);
    }
}

// The same for rows of at most kLnWavePasses * 512 values: one wavefront per
// step (four per workgroup), the row read once into registers (lane l holds
// values 512 p + 8 l .. +7 of each pass p), the statistics by wavefront
// reductions, no LDS or barriers.
constexpr int kLnWavePasses = 4;
__global__ __launch_bounds__(256) void layer_norm_digits_wave_kernel(const float *x, const float *weight,
                                                                     const float *bias, uint32_t width,
                                                                     uint32_t tokens, float eps, uint8_t *digits,
                                                                     float *mult) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t t = blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint32_t padded = (tokens + kTokenTile - 1) / kTokenTile * kTokenTile;
    if (t >= padded) return;  // (whole wavefronts)
    const bool real = t < tokens;
    const float *row = x + (size_t)(real ? t : 0) * width;
    const uint32_t gpr = width >> 6;
    float v[kLnWavePasses][8];
    float sum = 0.0f;
#pragma unroll
    for (int p = 0; p < kLnWavePasses; ++p) {
        const uint32_t e = 512 * p + 8 * lane;
        const bool in_row = e < width;
        load8(row + (in_row ? e : 0), v[p]);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v[p][i] = in_row ? v[p][i] : 0.0f;
            sum += v[p][i];
        }
    }
    const float mean = dev::wave_sum(sum) / (float)width;
    float squares = 0.0f;
#pragma unroll
    for (int p = 0; p < kLnWavePasses; ++p) {
        const bool in_row = 512 * p + 8 * lane < width;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float centered = v[p][i] - mean;
            squares += in_row ? centered * centered : 0.0f;
        }
    }
    const float inverse_std = 1.0f / sqrtf(dev::wave_sum(squares) / (float)width + eps);
#pragma unroll
    for (int p = 0; p < kLnWavePasses; ++p) {
        const uint32_t e = 512 * p + 8 * lane;
        if (512 * p >= width) break;  // (uniform)
        const bool in_row = e < width;
        float w[8], b[8];
        load8(weight + (in_row ? e : 0), w);
        load8(bias + (in_row ? e : 0), b);
        float y[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] = real ? (v[p][i] - mean) * inverse_std * w[i] + b[i] : 0.0f;
        if (in_row) encode_digits8(y, t / kTokenTile, t % kTokenTile, e, gpr, digits, mult);
    }
}

template <Prep M>
__global__ __launch_bounds__(64) void prep_batch_kernel(const PrepArgs a) {
    const uint32_t t = blockIdx.y;
    const uint32_t lane = threadIdx.x;
    const uint32_t e = blockIdx.x * kPrepValues + lane * 8;
    const uint32_t gpr = a.k >> 6;
    const uint32_t tile = t / kTokenTile;
    const uint32_t tt = t % kTokenTile;
    const bool real = t < a.tokens;
    const bool in_row = e < a.k;  // (whole groups: K is a multiple of 64)
    float v[8];
    input8<M>(a, real ? t : 0, in_row ? e : 0, v);  // padding tokens read token 0 and drop it
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = real && in_row ? v[i] : 0.0f;
    if constexpr (M == Prep::RmsNorm) {
        float w[8];
        load8(a.norm + (in_row ? e : 0), w);
        if (a.slices && real && in_row) store8(a.x_out + (size_t)t * a.k + e, v);
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) ss = __fadd_rn(ss, __fmul_rn(v[i], v[i]));
        ss = dev::wave_sum(ss);
        if (lane == 0) a.ss[(size_t)t * gridDim.x + blockIdx.x] = ss;
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = __fmul_rn(v[i], w[i]);
    }
    if (!in_row) return;
    encode_digits8(v, tile, tt, e, gpr, a.digits, a.mult);
}

}  // namespace

namespace {

// Layout of a batch activation buffer: digit planes, multipliers, then the
// RMSNorm sums of squares [token][ss_parts].
uint32_t ss_parts_of(uint32_t cols) { return (cols + kPrepValues - 1) / kPrepValues; }

float *mult_of(void *digits, uint32_t tokens, uint32_t cols) {
    const size_t tiles = (tokens + kTokenTile - 1) / kTokenTile;
    return reinterpret_cast<float *>(static_cast<uint8_t *>(digits) + tiles * (cols / 64) * kGroupBytes);
}

float *ss_of(void *digits, uint32_t tokens, uint32_t cols) {
    const size_t tiles = (tokens + kTokenTile - 1) / kTokenTile;
    return mult_of(digits, tokens, cols) + tiles * (cols / 64) * kTokenTile;
}

}  // namespace

size_t batch_digit_bytes(uint32_t tokens, uint32_t cols) {
    const size_t tiles = (tokens + kTokenTile - 1) / kTokenTile;
    const size_t groups = cols / 64;
    return tiles * groups * kGroupBytes + tiles * groups * kTokenTile * sizeof(float) +
           tiles * kTokenTile * ss_parts_of(cols) * sizeof(float) + 256;
}

hipError_t launch_layer_norm_digits(hipStream_t s, const float *x, const float *weight, const float *bias,
                                    uint32_t width, uint32_t tokens, float eps, void *digits) {
    if (!tokens || width % 64) return hipErrorInvalidValue;
    const uint32_t tiles = (tokens + kTokenTile - 1) / kTokenTile;
    uint8_t *d = static_cast<uint8_t *>(digits);
    float *m = mult_of(digits, tokens, width);
    // The wavefront form loads 16 bytes at a time from each row.
    const bool aligned = (((uintptr_t)x | (uintptr_t)weight | (uintptr_t)bias) & 15u) == 0 && width % 4 == 0;
    if (width <= 512u * kLnWavePasses && aligned)
        layer_norm_digits_wave_kernel<<<tiles * kTokenTile / 4, 256, 0, s>>>(x, weight, bias, width, tokens, eps, d,
                                                                             m);
    else
        layer_norm_digits_kernel<<<tiles * kTokenTile, 256, 0, s>>>(x, weight, bias, width, tokens, eps, d, m);
    return hipGetLastError();
}

hipError_t launch_prep_batch(hipStream_t s, const GemvInput &in, uint32_t tokens, uint32_t cols, void *digits,
                             const PartialSums *sums) {
    const uint32_t tiles = (tokens + kTokenTile - 1) / kTokenTile;
    PrepArgs p{};
    p.x = in.x;
    p.norm = in.norm;
    p.k = cols;
    p.tokens = tokens;
    p.digits = static_cast<uint8_t *>(digits);
    p.mult = mult_of(digits, tokens, cols);
    p.ss = ss_of(digits, tokens, cols);
    Prep form = in.mode == GemvInput::RmsNorm ? Prep::RmsNorm : Prep::F32;
    if (in.gelu_bias) {
        if (in.mode != GemvInput::F32 || (sums && sums->slices)) return hipErrorInvalidValue;
        p.bias = in.gelu_bias;
        form = Prep::BiasGelu;
    }
    if (in.mode != GemvInput::F32 && in.mode != GemvInput::RmsNorm) return hipErrorInvalidValue;
    if (form == Prep::RmsNorm && ss_parts_of(cols) > kTokenTile) return hipErrorInvalidValue;  // K > 8192
    if (sums && sums->slices) {
        if (sums->slices > kMaxSlices || !sums->part) return hipErrorInvalidValue;
        p.part = sums->part;
        p.slices = sums->slices;
        if (sums->pairs) {
            if (in.mode != GemvInput::F32 || sums->rows != 2 * cols) return hipErrorInvalidValue;
            form = Prep::Pairs;
        } else {
            if (in.mode != GemvInput::RmsNorm || sums->rows != cols || !sums->x_out) return hipErrorInvalidValue;
            p.x_out = sums->x_out;
        }
        p.part_n = sums->rows;
    }
    const dim3 grid(ss_parts_of(cols), tiles * kTokenTile);
    switch (form) {
    case Prep::F32: prep_batch_kernel<Prep::F32><<<grid, 64, 0, s>>>(p); break;
    case Prep::RmsNorm: prep_batch_kernel<Prep::RmsNorm><<<grid, 64, 0, s>>>(p); break;
    case Prep::Pairs: prep_batch_kernel<Prep::Pairs><<<grid, 64, 0, s>>>(p); break;
    case Prep::BiasGelu: prep_batch_kernel<Prep::BiasGelu><<<grid, 64, 0, s>>>(p); break;
    }
    return hipGetLastError();
}

namespace {

// Split-form plan: TW tiles per wavefront, chunks of KC groups, K slices.
// tw == 0: no split form for this shape (an odd number of groups).
struct SplitPlan {
    int tw = 0, kc = 4;
    uint32_t slices = 1, slice_groups = 0;
};

// `tiles`: the 16-token tiles of the call, which multiply the workgroups as
// the K slices do (the decoder's slice counts are planned for one tile).
SplitPlan split_plan(const Matrix &w, uint32_t tiles = 1) {
    SplitPlan p;
    const uint32_t gpr = w.cols / 64;
    if (gpr % 2u) return p;
    // Chunks of 4 groups, or of 2 where the group count is not a multiple of
    // 4 (the audio tower's 896-wide rows: 14 groups).
    p.kc = gpr % 4u ? 2 : 4;
    const uint32_t row_tiles = (w.rows + kRowTile - 1) / kRowTile;
    // Two tiles per wavefront once that still leaves 64 workgroups, else one.
    p.tw = row_tiles >= 4u * 2u * 64u ? 2 : 1;
    const uint32_t chunks = gpr / (uint32_t)p.kc;
    const uint32_t blocks = (row_tiles + 4u * p.tw - 1) / (4u * p.tw) * (tiles ? tiles : 1);
    // K slices: about 512 workgroups in all and at most about 4 chunks in
    // a row per workgroup (its chunks are one memory round trip each), a
    // divisor of the chunk count, at most kMaxSlices.
    uint32_t want = std::max((512u + blocks - 1) / blocks, (chunks + 3) / 4);
    p.slices = 1;
    for (uint32_t c = 1; c <= chunks && c <= want && c <= kMaxSlices; ++c)
        if (chunks % c == 0) p.slices = c;
    p.slice_groups = gpr / p.slices;
    return p;
}

template <int BPG>
void launch_split_bpg(hipStream_t s, const SplitPlan &plan, const SplitArgs &a, dim3 grid) {
    // Chunks of 2 or 4 groups (split_plan), one or two row tiles per wave.
    if (plan.kc == 2) {
        if (plan.tw == 2) gemv_split_kernel<2, 2, BPG><<<grid, 256, 0, s>>>(a);
        else gemv_split_kernel<1, 2, BPG><<<grid, 256, 0, s>>>(a);
    } else if (plan.tw == 2) {
        gemv_split_kernel<2, 4, BPG><<<grid, 256, 0, s>>>(a);
    } else {
        gemv_split_kernel<1, 4, BPG><<<grid, 256, 0, s>>>(a);
    }
}

template <int BPG>
void launch_split_multi_bpg(hipStream_t s, const SplitPlan &plan, const SplitMulti &m, dim3 grid) {
    // Chunks of 2 or 4 groups (split_plan), one or two row tiles per wave.
    if (plan.kc == 2) {
        if (plan.tw == 2) gemv_split_multi_kernel<2, 2, BPG><<<grid, 256, 0, s>>>(m);
        else gemv_split_multi_kernel<1, 2, BPG><<<grid, 256, 0, s>>>(m);
    } else if (plan.tw == 2) {
        gemv_split_multi_kernel<2, 4, BPG><<<grid, 256, 0, s>>>(m);
    } else {
        gemv_split_multi_kernel<1, 4, BPG><<<grid, 256, 0, s>>>(m);
    }
}

void launch_split(hipStream_t s, const SplitPlan &plan, const SplitArgs &a, uint32_t tiles, int format) {
    const uint32_t row_tiles = (a.n + kRowTile - 1) / kRowTile;
    const dim3 grid((row_tiles + 4u * plan.tw - 1) / (4u * plan.tw), plan.slices, tiles);
    if (format == QWH_FORMAT_Q5) {
        // (A slice is a whole number of chunks.)
        if (plan.kc == 2) {
            if (plan.tw == 2) gemv_split_q5_kernel<2, 2><<<grid, 256, 0, s>>>(a);
            else gemv_split_q5_kernel<1, 2><<<grid, 256, 0, s>>>(a);
        } else {
            if (plan.tw == 2) gemv_split_q5_kernel<2, 4><<<grid, 256, 0, s>>>(a);
            else gemv_split_q5_kernel<1, 4><<<grid, 256, 0, s>>>(a);
        }
    } else if (format == QWH_FORMAT_Q8) {
        launch_split_bpg<64>(s, plan, a, grid);
    } else {
        launch_split_bpg<32>(s, plan, a, grid);
    }
}

// Formats with a matrix-core form: q4, q8, and q5 in the split form only
// (its 40-byte groups are not 16-byte pieces for the unsplit kernel's LDS
// transpose).
bool batch_format(int format) {
    return format == QWH_FORMAT_Q4 || format == QWH_FORMAT_Q8 || format == QWH_FORMAT_Q5;
}

SplitArgs split_args(const void *digits, const Matrix &w, uint32_t tokens, const SplitPlan &plan,
                     const BatchNorm &norm) {
    SplitArgs a{};
    a.digits = static_cast<const uint8_t *>(digits);
    a.mult = mult_of(const_cast<void *>(digits), tokens, w.cols);
    if (norm.rms) {
        a.ss = ss_of(const_cast<void *>(digits), tokens, w.cols);
        a.ss_parts = ss_parts_of(w.cols);
        a.eps = norm.eps;
    }
    a.scales = reinterpret_cast<const uint16_t *>(w.scales);
    a.data = w.data;
    a.n = w.rows;
    a.k = w.cols;
    a.tokens = tokens;
    a.slice_groups = plan.slice_groups;
    return a;
}

}  // namespace

bool gemv_batch_supported(const Matrix &w) {
    if (!batch_format(w.format) || w.cols % 64) return false;
    if (w.format != QWH_FORMAT_Q5) return true;
    return split_plan(w).tw != 0;  // (q5: the split form, an even number of groups)
}

uint32_t batch_slices(const Matrix &w) {
    if (!batch_format(w.format)) return 0;
    const SplitPlan p = split_plan(w);
    return p.tw ? p.slices : 0;
}

size_t batch_partial_bytes(uint32_t tokens, const Matrix &w) {
    return (size_t)batch_slices(w) * tokens * w.rows * sizeof(float);
}

hipError_t launch_gemv_batch_parts(hipStream_t s, const void *digits, const Matrix &w, uint32_t tokens,
                                   float *partials, const BatchNorm &norm, uint32_t *slices_used) {
    if (!batch_format(w.format)) return hipErrorNotSupported;
    const SplitPlan plan = split_plan(w, slices_used ? (tokens + kTokenTile - 1) / kTokenTile : 1);
    if (slices_used) *slices_used = plan.slices;
    if (!plan.tw || !partials) return hipErrorInvalidValue;
    if (norm.rms && ss_parts_of(w.cols) > kTokenTile) return hipErrorInvalidValue;
    SplitArgs a = split_args(digits, w, tokens, plan, norm);
    a.part = partials;
    launch_split(s, plan, a, (tokens + kTokenTile - 1) / kTokenTile, w.format);
    return hipGetLastError();
}

hipError_t launch_gemv_batch_multi(hipStream_t s, const void *digits, const Matrix *const *w, float *const *out,
                                   uint32_t count, uint32_t tokens) {
    if (count == 0 || count > (uint32_t)kMaxMulti || tokens == 0) return hipErrorInvalidValue;
    const uint32_t tiles = (tokens + kTokenTile - 1) / kTokenTile;
    const SplitPlan plan = split_plan(*w[0], tiles);
    if (!plan.tw || plan.slices != 1 || (w[0]->format != QWH_FORMAT_Q4 && w[0]->format != QWH_FORMAT_Q8))
        return hipErrorNotSupported;
    SplitMulti m{};
    m.count = count;
    uint32_t blocks = 0;
    for (uint32_t i = 0; i < count; ++i) {
        const SplitPlan p = split_plan(*w[i], tiles);
        if (w[i]->format != w[0]->format || w[i]->cols != w[0]->cols || p.tw != plan.tw || p.kc != plan.kc ||
            p.slices != 1)
            return hipErrorNotSupported;
        m.m[i] = split_args(digits, *w[i], tokens, plan, BatchNorm{});
        m.m[i].out = out[i];
        const uint32_t row_tiles = (w[i]->rows + kRowTile - 1) / kRowTile;
        m.blocks[i] = (row_tiles + 4u * plan.tw - 1) / (4u * plan.tw);
        blocks += m.blocks[i];
    }
    const dim3 grid(blocks, 1, tiles);
    if (w[0]->format == QWH_FORMAT_Q8) launch_split_multi_bpg<64>(s, plan, m, grid);
    else launch_split_multi_bpg<32>(s, plan, m, grid);
    return hipGetLastError();
}

hipError_t launch_gemv_batch(hipStream_t s, const void *digits, const Matrix &w, uint32_t tokens, float *out,
                             const float *residual, bool pairs, float *partials, const BatchNorm &norm,
                             const float *bias) {
    if (!batch_format(w.format)) return hipErrorNotSupported;
    if (pairs && (w.rows & 1u)) return hipErrorInvalidValue;
    if (pairs && bias) return hipErrorInvalidValue;
    if (norm.rms && ss_parts_of(w.cols) > kTokenTile) return hipErrorInvalidValue;
    const uint32_t tiles = (tokens + kTokenTile - 1) / kTokenTile;
    const SplitPlan plan = split_plan(w, tiles);
    if (w.format == QWH_FORMAT_Q5 && !(plan.tw && (plan.slices == 1 || partials))) return hipErrorInvalidValue;
    if (plan.tw && (plan.slices == 1 || partials)) {
        SplitArgs a = split_args(digits, w, tokens, plan, norm);
        a.out = out;
        a.residual = residual;
        a.bias = bias;
        a.pairs = pairs ? 1u : 0u;
        if (plan.slices > 1) a.part = partials;
        launch_split(s, plan, a, tiles, w.format);
        if (plan.slices > 1) {
            const size_t items = (size_t)tokens * (pairs ? w.rows / 2 : w.rows);
            split_reduce_kernel<<<(uint32_t)((items + 255) / 256), 256, 0, s>>>(partials, plan.slices, tokens, w.rows,
                                                                               residual, out, pairs ? 1u : 0u, bias);
        }
        return hipGetLastError();
    }
    // An odd number of groups: the unsplit form, one tile per workgroup.
    BatchArgs a{};
    a.digits = static_cast<const uint8_t *>(digits);
    a.mult = mult_of(const_cast<void *>(digits), tokens, w.cols);
    if (norm.rms) {
        a.ss = ss_of(const_cast<void *>(digits), tokens, w.cols);
        a.ss_parts = ss_parts_of(w.cols);
        a.eps = norm.eps;
    }
    a.scales = reinterpret_cast<const uint16_t *>(w.scales);
    a.data = w.data;
    a.out = out;
    a.residual = residual;
    a.bias = bias;
    a.n = w.rows;
    a.k = w.cols;
    a.tokens = tokens;
    a.pairs = pairs ? 1u : 0u;
    const uint32_t row_tiles = (w.rows + kRowTile - 1) / kRowTile;
    const uint32_t gpr = w.cols / 64;
    // Groups per unit: 8, lowered to divide the row's groups.
    int gr = 8;
    while (gpr % (uint32_t)gr) gr >>= 1;
    const uint32_t units = gpr / (uint32_t)gr;
    const dim3 grid(row_tiles, tiles);
#define QWH_BATCH_CASE(G_, B_)                                                                       \
    if (gr == G_ && bpg == B_) {                                                                     \
        using S = BatchShape<1, G_, B_>;                                                             \
        /* Wavefronts: the largest divisor of the unit count within the cap and 64 KB of LDS. */     \
        uint32_t waves = 1;                                                                          \
        for (uint32_t c = 1; c <= (uint32_t)max_waves<1>() && c * S::WAVE_BYTES <= 65536u; ++c)      \
            if (units % c == 0) waves = c;                                                           \
        gemv_batch_kernel<1, G_, B_><<<grid, 64 * waves, waves * S::WAVE_BYTES, s>>>(a);             \
        return hipGetLastError();                                                                    \
    }
    const int bpg = w.format == QWH_FORMAT_Q8 ? 64 : 32;
    QWH_BATCH_CASE(8, 32) QWH_BATCH_CASE(4, 32) QWH_BATCH_CASE(2, 32) QWH_BATCH_CASE(1, 32)
    QWH_BATCH_CASE(8, 64) QWH_BATCH_CASE(4, 64) QWH_BATCH_CASE(2, 64) QWH_BATCH_CASE(1, 64)
#undef QWH_BATCH_CASE
    return hipErrorInvalidValue;
}

}  // namespace qwh
