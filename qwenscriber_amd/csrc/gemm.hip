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
//
// Two forms: this file's kernel runs two 256-thread workgroups per CU, every
// wavefront loading, decoding and multiplying; gemm_roles.hip's runs one
// 512-thread workgroup per CU whose wavefronts are split into loaders and
// multipliers. The plan takes the second for grids of at most one
// workgroup per CU when its estimate is lower.
#include "gemm_stage.h"

namespace qwh {
namespace {

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
// by an estimate of the launch's time (written to *est_us): the grid runs in
// waves of `per_cu` workgroups per CU, a group step taking `step_full` us
// when a CU holds that many and `step_alone` us when it holds one; each
// range past the first adds its partials' traffic (8 bytes per output, at
// about 6.5 TB/s) and the reduce launch. Counts that would put more than
// `max_items` workgroups in the grid are not taken. (Measured on MI355X over
// the configs' shapes, the estimate ranks the split counts in the measured
// order.) The smallest count wins a tie.
uint32_t gemm_splits(int cus, uint32_t tokens, const Matrix &w, uint32_t per_cu, double step_full,
                     double step_alone, uint64_t max_items, double *est_us) {
    const uint32_t units = (uint32_t)(cus > 0 ? cus : 256);
    const uint32_t tiles = ((w.rows + BN - 1) / BN) * ((tokens + BM - 1) / BM);
    const uint32_t groups = w.cols / BK;
    uint32_t most = groups / 2 < kMaxSplits ? groups / 2 : kMaxSplits;
    if (most < 1) most = 1;
    uint32_t best = 1;
    double best_us = 0.0;
    for (uint32_t s = 1; s <= most; ++s) {
        const uint64_t items = (uint64_t)tiles * s;
        if (s > 1 && items > max_items) break;
        const double steps = (double)((groups + s - 1) / s);
        const uint64_t waves = items / (per_cu * units), rest = items % (per_cu * units);
        double us = (double)waves * steps * step_full + (rest ? steps * (rest > units ? step_full : step_alone) : 0.0);
        if (s > 1) us += (double)tokens * w.rows * 4.0 * (s + 1) / 6.5e6 + 2.0;
        if (s == 1 || us < best_us) {
            best = s;
            best_us = us;
        }
    }
    *est_us = best_us;
    return best;
}

// The launch plan. Two forms of the kernel:
// - gemm_bf16_kernel, two 256-thread workgroups per CU (about 1.7 us per
//   group step with two on a CU, 1.0 us with one);
// - gemm_pc_kernel, one 512-thread workgroup per CU with the producer and
//   consumer roles split (about 0.9 us per group step), for grids of at most
//   one workgroup per CU.
// The form with the smaller estimate runs. With the first form and more
// tiles than the device holds at once (two workgroups per CU), the tiles
// past the last full wave would run as a nearly empty wave of their own:
// they are split into group ranges instead (at most one workgroup per CU,
// at most 4 ranges, each at least two groups long).
struct GemmPlan {
    uint32_t splits = 1, tail_splits = 0, full = 0, tiles_x = 0, tiles = 0;
    bool split_roles = false;
};

GemmPlan gemm_plan(int cus, uint32_t tokens, const Matrix &w) {
    GemmPlan p;
    const uint32_t units = (uint32_t)(cus > 0 ? cus : 256);
    p.tiles_x = (w.rows + BN - 1) / BN;
    p.tiles = p.tiles_x * ((tokens + BM - 1) / BM);
    double shared_us = 0.0, split_us = 0.0;
    p.splits = gemm_splits(cus, tokens, w, 2, 1.7, 1.0, ~0ull, &shared_us);
    if (p.tiles <= units) {
        const uint32_t s = gemm_splits(cus, tokens, w, 1, 0.9, 0.9, units, &split_us);
        if (split_us <= shared_us) {
            p.splits = s;
            p.split_roles = true;
            return p;
        }
    }
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
    if (plan.split_roles)
        launch_gemm_roles(s, grid, args, w.format);
    else if (w.format == QWH_FORMAT_Q5)
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
