// The q4 / q5 / q8 GEMM's tile constants, its kernel arguments and the
// staging of one quantization group's tile (global loads, code decode, LDS
// stores), shared by the two forms of the kernel: gemm_bf16_kernel
// (gemm.hip) and gemm_pc_kernel (gemm_roles.hip).
#pragma once
#include "common.h"
#include "device.h"

namespace qwh {

struct GemmArgs {
    const uint16_t *x;       // M x K bf16
    const uint16_t *scales;  // N x K/64 f16
    const uint8_t *data;     // N x K/64 groups of 32 (q4) or 40 (q5) bytes
    float *out;              // M x N, or splits x M x N partials
    uint32_t m, n, k;
    uint32_t splits;
    // Tail form (tail_splits > 0, one-dimensional grid): workgroups 0 ..
    // full - 1 take tiles 0 .. full - 1 whole (tile t = n tile t % tiles_x,
    // m tile t / tiles_x) and write `out`; the remaining tiles are split into
    // tail_splits group ranges each, written as 128 x 128 partial tiles to
    // `tail` ([tile - full][range][row][column]).
    uint32_t tail_splits, full, tiles_x;
    float *tail;
};

// Launches gemm_pc_kernel for `format` (QWH_FORMAT_Q4 / _Q5 / _Q8) on `grid`,
// 512 threads per workgroup.
void launch_gemm_roles(hipStream_t s, dim3 grid, const GemmArgs &a, int32_t format);

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // (native: stays in registers)

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int BK = 64;              // one quantization group
constexpr int LDS_STRIDE = BK + 8;  // bf16 elements per LDS row (padding against bank conflicts)


// Weight formats of the kernel: q4 (32-byte groups), q5 (40), q8 (64).
constexpr int kQ4 = 0, kQ5 = 1, kQ8 = 2;

// A group's tile data held in registers between its global loads and its
// LDS stores: 4 x 16 B of activations and the codes of half a group row per
// thread: 16 B (q4), 16 B and the 4 bytes of those 32 codes' fifth bits
// (q5), or 32 B (q8: codes, then codes2).
struct Staged {
    u32x4 a[4];
    u32x4 codes;
    u32x4 codes2;
    uint32_t fifth;
};
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Rows past the matrix (tokens past M, weight rows past N) load its last row:
// they only reach output rows or columns that are never stored. Every load
// is unconditional, so all of them are in flight together.
template <int F>
__device__ __forceinline__ void stage_load(const GemmArgs &a, Staged &st, uint32_t m0, uint32_t n0, uint32_t g,
                                           int tid) {
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int idx = tid + it * 256;  // 0..1023: 128 rows x 8 chunks of 8 bf16
        const uint32_t row = min(m0 + (idx >> 3), a.m - 1);
        const int col = (idx & 7) * 8;
        st.a[it] = *reinterpret_cast<const u32x4 *>(a.x + (size_t)row * a.k + g * BK + col);
    }
    const uint32_t row = min(n0 + (tid >> 1), a.n - 1);
    const int half = tid & 1;
    if constexpr (F == kQ5) {
        // A 40-byte group: the half row's nibbles are only 8-byte aligned.
        const uint8_t *grp = a.data + (size_t)row * (a.k / 64) * 40 + g * 40;
        const u32x2 lo = *reinterpret_cast<const u32x2 *>(grp + half * 16);
        const u32x2 hi = *reinterpret_cast<const u32x2 *>(grp + half * 16 + 8);
        st.codes = u32x4{lo.x, lo.y, hi.x, hi.y};
        st.fifth = *reinterpret_cast<const uint32_t *>(grp + 32 + half * 4);
    } else if constexpr (F == kQ8) {
        // A 64-byte group: the half row is 32 bytes.
        const uint8_t *grp = a.data + (size_t)row * a.k + g * 64 + half * 32;
        st.codes = *reinterpret_cast<const u32x4 *>(grp);
        st.codes2 = *reinterpret_cast<const u32x4 *>(grp + 16);
    } else {
        st.codes = *reinterpret_cast<const u32x4 *>(a.data + (size_t)row * (a.k / 2) + g * 32 + half * 16);
    }
}

// The thread's 32 codes decoded to the bf16 of u - 8 (q5: u - 16, q8:
// u - 128), two per word: packed[j] holds codes 2j and 2j + 1.
template <int F>
__device__ __forceinline__ void stage_decode(const Staged &st, uint32_t (&packed)[16]) {
    // (The codes count as changed here, so their decode is not moved up to
    // their load: using a load's value waits for every load issued before it.)
    u32x4 codes = st.codes;
    asm volatile("" : "+v"(codes));
    const uint32_t w[4] = {codes.x, codes.y, codes.z, codes.w};
    if constexpr (F == kQ8) {
        u32x4 codes2 = st.codes2;
        asm volatile("" : "+v"(codes2));
        const uint32_t w8[8] = {codes.x, codes.y, codes.z, codes.w, codes2.x, codes2.y, codes2.z, codes2.w};
#pragma unroll
        for (int d = 0; d < 8; ++d) {
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                // Bytes 2p and 2p + 1 of the word: codes 4d + 2p, 4d + 2p + 1;
                // a byte converts to f32 exactly, minus 128 exactly.
                const float c0 = (float)((w8[d] >> (16 * p)) & 0xffu) - 128.0f;
                const float c1 = (float)((w8[d] >> (16 * p + 8)) & 0xffu) - 128.0f;
                packed[2 * d + p] = (__float_as_uint(c0) >> 16) | (__float_as_uint(c1) & 0xffff0000u);
            }
        }
    } else if constexpr (F == kQ5) {
        uint32_t fifth = st.fifth;
        asm volatile("" : "+v"(fifth));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                // Codes 8i + 2p (low nibble of byte p) and 8i + 2p + 1; their
                // fifth bits are bits 8i + 2p and 8i + 2p + 1 of the word.
                const int c0 = (int)(((w[i] >> (8 * p)) & 0xfu) | (((fifth >> (8 * i + 2 * p)) & 1u) << 4)) - 16;
                const int c1 = (int)(((w[i] >> (8 * p + 4)) & 0xfu) | (((fifth >> (8 * i + 2 * p + 1)) & 1u) << 4)) - 16;
                packed[i * 4 + p] = (__float_as_uint((float)c0) >> 16) | (__float_as_uint((float)c1) & 0xffff0000u);
            }
        }
    } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t sw = w[i] ^ 0x88888888u;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            // Nibbles 2p, 2p+1 of the dword are weights 8i + 2p, +1; the
            // sign-extended nibble of u ^ 8 is u - 8, exact in bf16 (the top
            // half of its f32).
            const int c0 = (int)(sw << (28 - 8 * p)) >> 28;
            const int c1 = (int)(sw << (24 - 8 * p)) >> 28;
            packed[i * 4 + p] = (__float_as_uint((float)c0) >> 16) | (__float_as_uint((float)c1) & 0xffff0000u);
        }
    }
    }
}

// Activations as they are, decoded codes, into one LDS buffer.
__device__ __forceinline__ void stage_write(const Staged &st, const uint32_t (&packed)[16], uint16_t *lds_a,
                                            uint16_t *lds_b, int tid) {
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int idx = tid + it * 256;
        const int row = idx >> 3;
        const int col = (idx & 7) * 8;
        *reinterpret_cast<u32x4 *>(&lds_a[row * LDS_STRIDE + col]) = st.a[it];
    }
    const int row = tid >> 1;
    const int half = tid & 1;
    u32x4 *dst = reinterpret_cast<u32x4 *>(&lds_b[row * LDS_STRIDE + half * 32]);
#pragma unroll
    for (int q = 0; q < 4; ++q) dst[q] = u32x4{packed[q * 4 + 0], packed[q * 4 + 1], packed[q * 4 + 2], packed[q * 4 + 3]};
}

template <int F>
__device__ __forceinline__ void stage_store(const Staged &st, uint16_t *lds_a, uint16_t *lds_b, int tid) {
    uint32_t packed[16];
    stage_decode<F>(st, packed);
    stage_write(st, packed, lds_a, lds_b, tid);
}

}  // namespace
}  // namespace qwh
