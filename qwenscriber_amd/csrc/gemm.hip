// q4 GEMM with bf16 activations on the bf16 MFMA units: the prefill /
// audio-token product of kernels.zig:118-158 with tokens = M > 1.
//
// out[m][n] = sum_k x[m][k] * (u[n][k] - 8) * s[n][k/64]
//
// The codes (u - 8, in [-8, 7]) are exact in bf16, so the MFMA multiplies the
// exact decoded integers by the exact bf16 activations; each 64-wide group's
// partial product is accumulated in f32 on its own and then scaled by the
// group's f16 scale (folding the scale into bf16 weights would round it).
//
// Tiling: a 256-thread workgroup computes a 128 x 128 tile of out; each wave a
// 64 x 64 quarter as 2 x 2 tiles of v_mfma_f32_32x32x16_bf16. Per group, the
// activation tile (128 x 64 bf16) and the decoded weight tile (128 x 64 bf16)
// are staged through LDS.
#include "common.h"
#include "device.h"

namespace qwh {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int BK = 64;        // one quantization group
constexpr int LDS_STRIDE = BK + 8;  // bf16 elements per LDS row (padding against bank conflicts)

struct GemmArgs {
    const uint16_t *x;       // M x K bf16
    const uint16_t *scales;  // N x K/64 f16
    const uint8_t *data;     // N x K/2 q4 codes
    float *out;              // M x N
    uint32_t m, n, k;
};

__global__ __launch_bounds__(256) void gemm_q4_bf16_kernel(const GemmArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t lds_a[BM * LDS_STRIDE];
    __shared__ __attribute__((aligned(16))) uint16_t lds_b[BN * LDS_STRIDE];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1;  // wave's 64-row half of the tile
    const int wn = wave & 1;   // wave's 64-column half
    const uint32_t n0 = blockIdx.x * BN;
    const uint32_t m0 = blockIdx.y * BM;
    const uint32_t groups = a.k / BK;
    const uint32_t gpr = groups;

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

    // MFMA operand coordinates (32x32x16 layout): lane -> row/col l % 32,
    // k block 8 * (l / 32).
    const int li = lane & 31;
    const int kb = (lane >> 5) * 8;

    for (uint32_t g = 0; g < groups; ++g) {
        // Stage activations: 128 rows x 64 bf16 = 128 B per row, 16 B per
        // thread-load, 4 loads per thread.
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const int idx = tid + it * 256;  // 0..1023
            const int row = idx >> 3;
            const int col = (idx & 7) * 8;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (m0 + row < a.m)
                v = *reinterpret_cast<const uint4 *>(a.x + (size_t)(m0 + row) * a.k + g * BK + col);
            *reinterpret_cast<uint4 *>(&lds_a[row * LDS_STRIDE + col]) = v;
        }
        // Stage decoded weights: row = tid / 2, 32 codes (16 bytes) per thread.
        {
            const int row = tid >> 1;
            const int half = tid & 1;
            uint4 codes = make_uint4(0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u);
            if (n0 + row < a.n)
                codes = *reinterpret_cast<const uint4 *>(a.data + (size_t)(n0 + row) * (a.k / 2) + g * 32 + half * 16);
            const uint32_t w[4] = {codes.x, codes.y, codes.z, codes.w};
            uint32_t packed[16];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t sw = w[i] ^ 0x88888888u;
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    // Nibbles 2p, 2p+1 of the dword are weights 8i + 2p, +1;
                    // the sign-extended nibble of u ^ 8 is u - 8.
                    const int c0 = (int)(sw << (28 - 8 * p)) >> 28;
                    const int c1 = (int)(sw << (24 - 8 * p)) >> 28;
                    const uint32_t b0 = __float_as_uint((float)c0) >> 16;
                    const uint32_t b1 = __float_as_uint((float)c1) >> 16;
                    packed[i * 4 + p] = b0 | (b1 << 16);
                }
            }
            uint4 *dst = reinterpret_cast<uint4 *>(&lds_b[row * LDS_STRIDE + half * 32]);
#pragma unroll
            for (int q = 0; q < 4; ++q)
                dst[q] = make_uint4(packed[q * 4 + 0], packed[q * 4 + 1], packed[q * 4 + 2], packed[q * 4 + 3]);
        }
        __syncthreads();

        f32x16 part[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) part[i][j] = f32x16{};
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            bf16x8 fa[2], fb[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int row = wm * 64 + i * 32 + li;
                fa[i] = *reinterpret_cast<const bf16x8 *>(&lds_a[row * LDS_STRIDE + ks * 16 + kb]);
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int row = wn * 64 + j * 32 + li;
                fb[j] = *reinterpret_cast<const bf16x8 *>(&lds_b[row * LDS_STRIDE + ks * 16 + kb]);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    part[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], part[i][j], 0, 0, 0);
        }
        // Scale each group's partial product by its weight row's scale: in the
        // 32x32 output layout every value a lane holds lies in column l % 32.
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t n = n0 + wn * 64 + j * 32 + li;
            const float s = n < a.n ? dev::f16_bits_to_f32(a.scales[(size_t)n * gpr + g]) : 0.0f;
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = fmaf(s, part[i][j][r], acc[i][j][r]);
        }
        __syncthreads();
    }

    // Store: value r of a lane is row 8 * (r / 4) + 4 * (l / 32) + r % 4 of the
    // 32x32 tile, column l % 32.
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t n = n0 + wn * 64 + j * 32 + li;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t m = m0 + wm * 64 + i * 32 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
                if (m < a.m && n < a.n) a.out[(size_t)m * a.n + n] = acc[i][j][r];
            }
        }
    }
}

}  // namespace

hipError_t launch_gemm_q4_bf16(hipStream_t s, const uint16_t *x, const Matrix &w, uint32_t tokens,
                               float *out) {
    GemmArgs args{};
    args.x = x;
    args.scales = reinterpret_cast<const uint16_t *>(w.scales);
    args.data = w.data;
    args.out = out;
    args.m = tokens;
    args.n = w.rows;
    args.k = w.cols;
    dim3 grid((w.rows + BN - 1) / BN, (tokens + BM - 1) / BM);
    gemm_q4_bf16_kernel<<<grid, 256, 0, s>>>(args);
    return hipGetLastError();
}

}  // namespace qwh
