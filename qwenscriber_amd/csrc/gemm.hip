// q4 / q5 / q8 GEMM with bf16 activations on the bf16 MFMA units: the
// prefill / audio-token product of kernels.zig:118-158 with tokens = M > 1.
//
// out[m][n] = sum_k x[m][k] * (u[n][k] - bias) * s[n][k/64]
//
// The codes (q4: u - 8 in [-8, 7]; q5: u - 16 in [-16, 15], the fifth bit of
// each code in its group's last 8 bytes, quant.zig:253-269; q8: u - 128 in
// [-128, 127], quant.zig:270-275, 336-340) are exact in bf16, so the MFMA
// multiplies the exact decoded integers by the exact bf16 activations; each
// 64-wide group's partial product is accumulated in f32 on its own and then
// scaled by the group's f16 scale (folding the scale into bf16 weights would
// round it).
//
// Tiling: a 256-thread workgroup computes a 128 x 128 tile of out; each wave a
// 64 x 64 quarter as 2 x 2 tiles of v_mfma_f32_32x32x16_bf16. The K loop runs
// over quantization groups and is software pipelined: while group g is
// multiplied out of one LDS buffer, group g+1's activations and codes wait in
// registers to be written (codes decoded to bf16) into the other buffer
// before the iteration's single barrier, and group g+2's are in flight from
// global memory. Within an iteration the decode and the scale FMAs (of the
// other 32-row half of the wave's tile) run between the MFMAs.
//
// Split K: when the tiles alone cannot fill the device (few tokens, or few
// weight rows), grid.z splits the groups into ranges; each range writes a
// partial tile and a second kernel adds the ranges in order (deterministic).
// When there are a little more tiles than the device holds at once, only
// the tiles past the last full wave are split (gemm_plan).
#include "common.h"
#include "device.h"

namespace qwh {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // (native: stays in registers)

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int BK = 64;              // one quantization group
constexpr int LDS_STRIDE = BK + 8;  // bf16 elements per LDS row (padding against bank conflicts)

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

template <int F>
__global__ __launch_bounds__(256, 2) void gemm_bf16_kernel(const GemmArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t lds_a[2][BM * LDS_STRIDE];
    __shared__ __attribute__((aligned(16))) uint16_t lds_b[2][BN * LDS_STRIDE];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1;  // wave's 64-row half of the tile
    const int wn = wave & 1;   // wave's 64-column half
    uint32_t tx = blockIdx.x, ty = blockIdx.y, z = blockIdx.z, ranges = a.splits, tile = 0;
    bool partial_tile = false;
    if (a.tail_splits) {
        tile = blockIdx.x;
        z = 0;
        ranges = 1;
        if (tile >= a.full) {
            const uint32_t j = tile - a.full;
            tile = a.full + j / a.tail_splits;
            z = j % a.tail_splits;
            ranges = a.tail_splits;
            partial_tile = true;
        }
        tx = tile % a.tiles_x;
        ty = tile / a.tiles_x;
    }
    const uint32_t n0 = tx * BN;
    const uint32_t m0 = ty * BM;
    const uint32_t gpr = a.k / BK;
    const uint32_t g0 = z * gpr / ranges;
    const uint32_t g1 = (z + 1) * gpr / ranges;

    // MFMA operand coordinates (32x32x16 layout): lane -> row/col l % 32,
    // k block 8 * (l / 32).
    const int li = lane & 31;
    const int kb = (lane >> 5) * 8;
    // This lane's two output columns (one per 32-column MFMA tile).
    uint32_t ncol[2];
    const uint16_t *srow[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        ncol[j] = n0 + wn * 64 + j * 32 + li;
        srow[j] = a.scales + (size_t)min(ncol[j], a.n - 1) * gpr;
    }

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

    // Two groups in flight ahead of the one being multiplied: group g + 2's
    // loads are issued while g is multiplied and g + 1 waits in registers.
    Staged st0, st1;
    stage_load<F>(a, st0, m0, n0, g0, tid);
    stage_load<F>(a, st1, m0, n0, min(g0 + 1, g1 - 1), tid);
    stage_store<F>(st0, lds_a[0], lds_b[0], tid);
    __syncthreads();

    // Each group's partial product is scaled by its weight row's scale (in
    // the 32x32 output layout every value a lane holds lies in column l % 32)
    // on the vector ALUs, one FMA per output value. The two 32-row halves of
    // the wave's tile run half a group apart, so those FMAs always have
    // products in flight beside them: the MFMAs of group g's first half run
    // while the second half of group g - 1 (part1, s_prev) is scaled, those of
    // its second half while its first half is scaled. Each value is scaled
    // and summed in group order, as before the split.
    f32x16 part1[2] = {f32x16{}, f32x16{}};
    float s_prev[2] = {0.0f, 0.0f};

    // One group: loads for g + 2 into `next2` (its previous content, group
    // g, is already in LDS), multiply group g from LDS buffer `buf`, then
    // store group g + 1 (in `next1`) into the other buffer; group g + 1's
    // decode is spread between the MFMAs.
    // The scales of group g come from the step before, issued ahead of that
    // step's tile loads (waiting for a load waits for every older one, so
    // scales fetched in their own step would drain the tile prefetch).
    auto step = [&](uint32_t g, int buf, Staged &next2, const Staged &next1, const uint32_t (&s_now)[2],
                    uint32_t (&s_next)[2]) {
#pragma unroll
        for (int j = 0; j < 2; ++j) s_next[j] = srow[j][min(g + 1, g1 - 1)];
        // (Past the range: the last group again, never used.)
        stage_load<F>(a, next2, m0, n0, min(g + 2, g1 - 1), tid);

        const uint16_t *la = lds_a[buf];
        const uint16_t *lb = lds_b[buf];
        uint32_t packed[16];
        stage_decode<F>(next1, packed);
        float s[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            uint32_t bits = s_now[j];
            asm volatile("" : "+v"(bits));  // (converted here, not at its load)
            s[j] = dev::f16_bits_to_f32((uint16_t)bits);
        }
        // The weight operands serve both halves: q4 reads them once into
        // registers; q5 and q8 (whose staging and decode hold more
        // registers) read them again for the second half rather than spill.
        constexpr bool kLazyB = F != kQ4;
        auto read_b = [&](int ks, int j) {
            return *reinterpret_cast<const bf16x8 *>(&lb[(wn * 64 + j * 32 + li) * LDS_STRIDE + ks * 16 + kb]);
        };
        bf16x8 fb[BK / 16][2];
        if constexpr (!kLazyB) {
#pragma unroll
            for (int ks = 0; ks < BK / 16; ++ks)
#pragma unroll
                for (int j = 0; j < 2; ++j) fb[ks][j] = read_b(ks, j);
        }
        f32x16 part0[2];
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const bf16x8 fa = *reinterpret_cast<const bf16x8 *>(&la[(wm * 64 + li) * LDS_STRIDE + ks * 16 + kb]);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                part0[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa, kLazyB ? read_b(ks, j) : fb[ks][j],
                                                                 ks == 0 ? f32x16{} : part0[j], 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[1][j][r] = fmaf(s_prev[j], part1[j][r], acc[1][j][r]);
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const bf16x8 fa = *reinterpret_cast<const bf16x8 *>(&la[(wm * 64 + 32 + li) * LDS_STRIDE + ks * 16 + kb]);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                part1[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa, kLazyB ? read_b(ks, j) : fb[ks][j],
                                                                 ks == 0 ? f32x16{} : part1[j], 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[0][j][r] = fmaf(s[j], part0[j][r], acc[0][j][r]);
        // Scheduling: each of the 16 MFMAs followed by up to six vector-ALU
        // instructions (the decode and the FMAs), as their operands allow
        // (measured against two, ten and the compiler's own order).
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // VALU
        }
        stage_write(next1, packed, lds_a[buf ^ 1], lds_b[buf ^ 1], tid);
        s_prev[0] = s[0];
        s_prev[1] = s[1];
        __syncthreads();
    };
    // Unrolled by two so the staging registers are addressed statically.
    uint32_t sc0[2], sc1[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) sc0[j] = srow[j][g0];
    uint32_t g = g0;
    for (; g + 1 < g1; g += 2) {
        step(g, 0, st0, st1, sc0, sc1);
        step(g + 1, 1, st1, st0, sc1, sc0);
    }
    if (g < g1) step(g, 0, st0, st1, sc0, sc1);
    // The last group's second half.
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[1][j][r] = fmaf(s_prev[j], part1[j][r], acc[1][j][r]);

    // Store: value r of a lane is row 8 * (r / 4) + 4 * (l / 32) + r % 4 of the
    // 32x32 tile, column l % 32.
    if (partial_tile) {
        // The whole 128 x 128 partial tile, rows and columns past the
        // matrix included (the reduce drops them).
        float *dst = a.tail + ((size_t)(tile - a.full) * a.tail_splits + z) * BM * BN;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = wm * 64 + i * 32 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
                    dst[row * BN + wn * 64 + j * 32 + li] = acc[i][j][r];
                }
        return;
    }
    float *out = a.out + (size_t)z * a.m * a.n;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t n = ncol[j];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t m = m0 + wm * 64 + i * 32 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
                if (m < a.m && n < a.n) out[(size_t)m * a.n + n] = acc[i][j][r];
            }
        }
    }
}

// out[i] = sum over ranges z (in order) of partial[z][i], four outputs per
// thread; every range's loads are issued before the first add.
constexpr uint32_t kMaxSplits = 8;

__global__ __launch_bounds__(256) void gemm_reduce_kernel(const float *partial, uint32_t splits, size_t count,
                                                          float *out) {
    const size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i >= count) return;
    if ((count & 3) == 0) {  // (every range's slice 16-byte aligned)
        float4 v[kMaxSplits];
#pragma unroll
        for (uint32_t z = 0; z < kMaxSplits; ++z)
            if (z < splits) v[z] = *reinterpret_cast<const float4 *>(partial + (size_t)z * count + i);
        float4 s = v[0];
#pragma unroll
        for (uint32_t z = 1; z < kMaxSplits; ++z)
            if (z < splits) {
                s.x += v[z].x;
                s.y += v[z].y;
                s.z += v[z].z;
                s.w += v[z].w;
            }
        *reinterpret_cast<float4 *>(out + i) = s;
        return;
    }
    for (size_t e = i; e < i + 4 && e < count; ++e) {
        float s = partial[e];
        for (uint32_t z = 1; z < splits; ++z) s += partial[(size_t)z * count + e];
        out[e] = s;
    }
}

// The tail tiles' partials, summed over their ranges in order into `out`
// (rows and columns inside the matrix only): 16 workgroups of 256 threads
// per tile, four consecutive columns per thread.
__global__ __launch_bounds__(256) void gemm_tail_reduce_kernel(const float *tail, uint32_t splits, uint32_t full,
                                                               uint32_t tiles_x, uint32_t m, uint32_t n, float *out) {
    const uint32_t t = blockIdx.x / 16;
    const uint32_t e = ((blockIdx.x % 16) * 256 + threadIdx.x) * 4;
    const uint32_t tile = full + t;
    const uint32_t mm = (tile / tiles_x) * BM + e / BN;
    const uint32_t nn = (tile % tiles_x) * BN + e % BN;
    if (mm >= m) return;
    const float *src = tail + (size_t)t * splits * BM * BN + e;
    float4 s = *reinterpret_cast<const float4 *>(src);
    for (uint32_t z = 1; z < splits; ++z) {
        const float4 v = *reinterpret_cast<const float4 *>(src + (size_t)z * BM * BN);
        s.x += v.x;
        s.y += v.y;
        s.z += v.z;
        s.w += v.w;
    }
    float *dst = out + (size_t)mm * n + nn;
    const float vals[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
    for (int c = 0; c < 4; ++c)
        if (nn + c < n) dst[c] = vals[c];
}

// Ranges of groups per tile (1 .. 8, each at least two groups long), chosen
// by an estimate of the launch's time: the grid runs in waves of two
// workgroups per CU, a group step taking about 1.7 us when a CU holds two
// workgroups and 1.0 us when it holds one; each range past the first adds
// its partials' traffic (8 bytes per output, at about 6.5 TB/s) and the
// reduce launch. (Measured on MI355X over the configs' shapes, the estimate
// ranks the split counts in the measured order.) The smallest count wins a
// tie.
uint32_t gemm_splits(int cus, uint32_t tokens, const Matrix &w) {
    const uint32_t units = (uint32_t)(cus > 0 ? cus : 256);
    const uint32_t tiles = ((w.rows + BN - 1) / BN) * ((tokens + BM - 1) / BM);
    const uint32_t groups = w.cols / BK;
    uint32_t most = groups / 2 < kMaxSplits ? groups / 2 : kMaxSplits;
    if (most < 1) most = 1;
    uint32_t best = 1;
    double best_us = 0.0;
    for (uint32_t s = 1; s <= most; ++s) {
        const uint64_t items = (uint64_t)tiles * s;
        const double steps = (double)((groups + s - 1) / s);
        const uint64_t waves = items / (2 * units), rest = items % (2 * units);
        double us = (double)waves * steps * 1.7 + (rest ? steps * (rest > units ? 1.7 : 1.0) : 0.0);
        if (s > 1) us += (double)tokens * w.rows * 4.0 * (s + 1) / 6.5e6 + 2.0;
        if (s == 1 || us < best_us) {
            best = s;
            best_us = us;
        }
    }
    return best;
}

// With more tiles than the device holds at once (two workgroups per CU),
// the tiles past the last full wave would run as a nearly empty wave of
// their own: they are split into group ranges instead (at most one
// workgroup per CU, at most 4 ranges, each at least two groups long).
struct GemmPlan {
    uint32_t splits = 1, tail_splits = 0, full = 0, tiles_x = 0, tiles = 0;
};

GemmPlan gemm_plan(int cus, uint32_t tokens, const Matrix &w) {
    GemmPlan p;
    const uint32_t units = (uint32_t)(cus > 0 ? cus : 256);
    p.tiles_x = (w.rows + BN - 1) / BN;
    p.tiles = p.tiles_x * ((tokens + BM - 1) / BM);
    p.splits = gemm_splits(cus, tokens, w);
    const uint32_t slots = 2 * units;
    if (p.splits == 1 && p.tiles > slots) {
        const uint32_t rem = p.tiles % slots;
        uint32_t ts = rem ? units / rem : 0;
        if (ts > 4) ts = 4;
        if (ts > w.cols / BK / 2) ts = w.cols / BK / 2;
        if (ts >= 2) {
            p.tail_splits = ts;
            p.full = p.tiles - rem;
        }
    }
    return p;
}

}  // namespace

size_t gemm_scratch_bytes(int cus, uint32_t tokens, const Matrix &w) {
    const GemmPlan p = gemm_plan(cus, tokens, w);
    if (p.tail_splits) return (size_t)(p.tiles - p.full) * p.tail_splits * BM * BN * sizeof(float);
    return p.splits > 1 ? (size_t)p.splits * tokens * w.rows * sizeof(float) : 0;
}

hipError_t launch_gemm_bf16(hipStream_t s, int cus, const uint16_t *x, const Matrix &w, uint32_t tokens,
                            float *out, void *scratch) {
    if (w.format != QWH_FORMAT_Q4 && w.format != QWH_FORMAT_Q5 && w.format != QWH_FORMAT_Q8)
        return hipErrorNotSupported;
    GemmArgs args{};
    args.x = x;
    args.scales = reinterpret_cast<const uint16_t *>(w.scales);
    args.data = w.data;
    args.m = tokens;
    args.n = w.rows;
    args.k = w.cols;
    const GemmPlan plan = gemm_plan(cus, tokens, w);
    args.splits = plan.splits;
    args.out = args.splits > 1 ? static_cast<float *>(scratch) : out;
    dim3 grid((w.rows + BN - 1) / BN, (tokens + BM - 1) / BM, args.splits);
    if (plan.tail_splits) {
        args.tail_splits = plan.tail_splits;
        args.full = plan.full;
        args.tiles_x = plan.tiles_x;
        args.tail = static_cast<float *>(scratch);
        grid = dim3(plan.full + (plan.tiles - plan.full) * plan.tail_splits);
    }
    if (w.format == QWH_FORMAT_Q5)
        gemm_bf16_kernel<kQ5><<<grid, 256, 0, s>>>(args);
    else if (w.format == QWH_FORMAT_Q8)
        gemm_bf16_kernel<kQ8><<<grid, 256, 0, s>>>(args);
    else
        gemm_bf16_kernel<kQ4><<<grid, 256, 0, s>>>(args);
    if (plan.tail_splits) {
        gemm_tail_reduce_kernel<<<(plan.tiles - plan.full) * 16, 256, 0, s>>>(
            args.tail, plan.tail_splits, plan.full, plan.tiles_x, tokens, w.rows, out);
    } else if (args.splits > 1) {
        const size_t count = (size_t)tokens * w.rows;
        gemm_reduce_kernel<<<(unsigned)((count + 1023) / 1024), 256, 0, s>>>(args.out, args.splits, count, out);
    }
    return hipGetLastError();
}

}  // namespace qwh
