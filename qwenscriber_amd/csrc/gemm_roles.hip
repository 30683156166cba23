// The producer / consumer form of the q4 / q5 / q8 GEMM with bf16
// activations (gemm.hip has the shared-role form, the plan that chooses
// between them, and the reduce kernels). Its own translation unit, so that
// the shared-role kernel's code is compiled as it is without it.
#include "gemm_stage.h"

namespace qwh {
namespace {

// Producer / consumer form of the same tile, one 512-thread workgroup per CU:
// wavefronts 0-3 only multiply and scale (each its 64 x 64 quarter, with
// the half-tile offset of gemm.hip's gemm_bf16_kernel), wavefronts 4-7 only
// load, decode and stage the next group into the other LDS buffer. A SIMD then holds one wavefront of
// each kind, so the decode's vector-ALU work and the loads' waits run beside
// the matrix-core work instead of between it. One barrier per group, as
// there; both kinds pass the same number of barriers. Each output value is
// scaled and summed in the same group order as gemm_bf16_kernel, so the two
// forms give the same bits.
template <int F>
__global__ __launch_bounds__(512, 1) void gemm_pc_kernel(const GemmArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t lds_a[2][BM * LDS_STRIDE];
    __shared__ __attribute__((aligned(16))) uint16_t lds_b[2][BN * LDS_STRIDE];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
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

    if (wave >= 4) {
        // Producers: thread pt stages what thread pt of gemm_bf16_kernel
        // stages. Group g + 2's loads go out before group g + 1 (loaded one
        // step earlier) is decoded and written.
        const int pt = tid - 256;
        Staged st0, st1;
        stage_load<F>(a, st0, m0, n0, g0, pt);
        stage_load<F>(a, st1, m0, n0, min(g0 + 1, g1 - 1), pt);
        stage_store<F>(st0, lds_a[0], lds_b[0], pt);
        __syncthreads();
        auto pstep = [&](uint32_t g, int buf, Staged &next2, const Staged &next1) {
            stage_load<F>(a, next2, m0, n0, min(g + 2, g1 - 1), pt);
            // (Past the range: the last group again, written to the buffer
            // nobody reads after the last step.)
            stage_store<F>(next1, lds_a[buf ^ 1], lds_b[buf ^ 1], pt);
            __syncthreads();
        };
        uint32_t g = g0;
        for (; g + 1 < g1; g += 2) {
            pstep(g, 0, st0, st1);
            pstep(g + 1, 1, st1, st0);
        }
        if (g < g1) pstep(g, 0, st0, st1);
        return;
    }

    const int wm = wave >> 1;
    const int wn = wave & 1;
    const int li = lane & 31;
    const int kb = (lane >> 5) * 8;
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
    f32x16 part1[2] = {f32x16{}, f32x16{}};
    float s_prev[2] = {0.0f, 0.0f};
    __syncthreads();
    auto cstep = [&](uint32_t g, int buf, const uint32_t (&s_now)[2], uint32_t (&s_next)[2]) {
#pragma unroll
        for (int j = 0; j < 2; ++j) s_next[j] = srow[j][min(g + 1, g1 - 1)];
        const uint16_t *la = lds_a[buf];
        const uint16_t *lb = lds_b[buf];
        float s[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            uint32_t bits = s_now[j];
            asm volatile("" : "+v"(bits));
            s[j] = dev::f16_bits_to_f32((uint16_t)bits);
        }
        bf16x8 fb[BK / 16][2];
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks)
#pragma unroll
            for (int j = 0; j < 2; ++j)
                fb[ks][j] = *reinterpret_cast<const bf16x8 *>(&lb[(wn * 64 + j * 32 + li) * LDS_STRIDE + ks * 16 + kb]);
        f32x16 part0[2];
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const bf16x8 fa = *reinterpret_cast<const bf16x8 *>(&la[(wm * 64 + li) * LDS_STRIDE + ks * 16 + kb]);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                part0[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa, fb[ks][j], ks == 0 ? f32x16{} : part0[j], 0, 0,
                                                                 0);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[1][j][r] = fmaf(s_prev[j], part1[j][r], acc[1][j][r]);
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const bf16x8 fa =
                *reinterpret_cast<const bf16x8 *>(&la[(wm * 64 + 32 + li) * LDS_STRIDE + ks * 16 + kb]);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                part1[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa, fb[ks][j], ks == 0 ? f32x16{} : part1[j], 0, 0,
                                                                 0);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[0][j][r] = fmaf(s[j], part0[j][r], acc[0][j][r]);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // VALU
        }
        s_prev[0] = s[0];
        s_prev[1] = s[1];
        __syncthreads();
    };
    uint32_t sc0[2], sc1[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) sc0[j] = srow[j][g0];
    uint32_t g = g0;
    for (; g + 1 < g1; g += 2) {
        cstep(g, 0, sc0, sc1);
        cstep(g + 1, 1, sc1, sc0);
    }
    if (g < g1) cstep(g, 0, sc0, sc1);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[1][j][r] = fmaf(s_prev[j], part1[j][r], acc[1][j][r]);

    if (partial_tile) {
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

}  // namespace

void launch_gemm_roles(hipStream_t s, dim3 grid, const GemmArgs &a, int32_t format) {
    if (format == QWH_FORMAT_Q5)
        gemm_pc_kernel<kQ5><<<grid, 512, 0, s>>>(a);
    else if (format == QWH_FORMAT_Q8)
        gemm_pc_kernel<kQ8><<<grid, 512, 0, s>>>(a);
    else
        gemm_pc_kernel<kQ4><<<grid, 512, 0, s>>>(a);
}

}  // namespace qwh
