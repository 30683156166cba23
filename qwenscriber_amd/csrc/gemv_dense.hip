// f16 and f32 weights: the Matrix.apply .f16 / .f32 arms (kernels.zig:160-206,
// linearF16 :82-112, linearF32 :54-80). out[t][r] = sum_k w[r][k] x[t][k],
// each f16 weight widened exactly to f32 (half_float.zig:20-23 fromF16), f32
// products and sums (the reference sums in dotF32's four-lane order,
// kernels.zig:38-51; this sum runs over a wavefront's lanes, within f32
// rounding of it). From eight tokens the matrix cores take the product:
// f32 with widened weights, or for f16 weights f16 operands that carry each
// activation to 2^-22 of its 64-value step's largest magnitude.
//
// HBM bound: the weights stream once per group of up to four tokens (fewer
// for rows too wide for four tokens' activations in LDS). Each workgroup forms its
// tokens' activations in LDS once (as they are, or after RMSNorm,
// math.zig:118-130), and its wavefronts walk outputs grid-stride. A row is
// read in chunks of four 16-byte slices per lane (8 f16 or 4 f32 values
// each): the first chunk is requested before the activations are formed,
// and each next chunk while the current one is multiplied by every token's
// activations. An output's row sums (gate and up with pairs, each token's)
// are reduced over the wavefront in one transposed butterfly. For f16 rows
// the activations of a slice's two 16-byte halves sit in two LDS planes so
// that the lanes' LDS reads are consecutive 16-byte words. Rows that are not
// whole 16-byte slices, or a plane that is not 16-byte aligned, take the
// element-wise form. Epilogues as the q4 GEMV: + residual, or siluMul of
// gate / up row pairs (kernels.zig:233-239).
#include "common.h"
#include "device.h"

namespace qwh {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // native: stays in registers

struct DenseArgs {
    const uint8_t *w;       // rows x cols f16 or f32, row major
    uint32_t rows, cols;
    uint32_t tokens;
    const float *x;         // tokens x cols
    const float *norm;      // RmsNorm form: cols weights
    float eps;
    float *out;             // tokens x rows (pairs: tokens x rows / 2)
    const float *residual;  // optional, tokens x rows (not with pairs); may alias out
    uint32_t pairs;
};

// The widest rows a workgroup of TOK tokens takes: one token's activations
// and partial sums may fill the 160 KiB of LDS a gfx950 workgroup can use;
// a group of several stays within 64 KiB, so that at least two workgroups
// share a CU (groups of eight tokens, or four at 98 KiB, measured slower on
// the 1.7B decoder's batch-16 step and prompt prefill than more passes over
// the weights with more wavefronts in flight).
constexpr uint32_t dense_lds_limit(int tok) { return tok == 1 ? 160u << 10 : 64u << 10; }
constexpr uint32_t dense_max_cols(int tok) {
    return (dense_lds_limit(tok) - 16u * (uint32_t)tok) / (4u * (uint32_t)tok);
}
static_assert(dense_max_cols(1) == kDenseMaxCols, "one token's activations fill the LDS");

template <bool Half>
__device__ __forceinline__ float dense_weight(const uint8_t *w, size_t i) {
    if constexpr (Half) return dev::f16_bits_to_f32(reinterpret_cast<const uint16_t *>(w)[i]);
    else return reinterpret_cast<const float *>(w)[i];
}

// Sum of one 16-byte slice's products with its activations: lo holds the
// first four (f16: values 0-3 of the slice, f32: all four), hi values 4-7.
template <bool Half>
__device__ __forceinline__ float slice_dot(const u32x4 v, const float4 lo, const float4 hi) {
    float s;
    if constexpr (Half) {
        s = dev::f16_bits_to_f32((uint16_t)(v.x & 0xffffu)) * lo.x;
        s = fmaf(dev::f16_bits_to_f32((uint16_t)(v.x >> 16)), lo.y, s);
        s = fmaf(dev::f16_bits_to_f32((uint16_t)(v.y & 0xffffu)), lo.z, s);
        s = fmaf(dev::f16_bits_to_f32((uint16_t)(v.y >> 16)), lo.w, s);
        s = fmaf(dev::f16_bits_to_f32((uint16_t)(v.z & 0xffffu)), hi.x, s);
        s = fmaf(dev::f16_bits_to_f32((uint16_t)(v.z >> 16)), hi.y, s);
        s = fmaf(dev::f16_bits_to_f32((uint16_t)(v.w & 0xffffu)), hi.z, s);
        s = fmaf(dev::f16_bits_to_f32((uint16_t)(v.w >> 16)), hi.w, s);
    } else {
        (void)hi;
        s = __uint_as_float(v.x) * lo.x;
        s = fmaf(__uint_as_float(v.y), lo.y, s);
        s = fmaf(__uint_as_float(v.z), lo.z, s);
        s = fmaf(__uint_as_float(v.w), lo.w, s);
    }
    return s;
}

// The first N sums of v, each over the wavefront, in one transposed
// butterfly: each of the first log2 N exchanges halves the values a lane
// holds (a lane keeps the half its lane bit selects and adds the other lane's
// copy of it), the rest add the one value left. Lane l ends with the sum of
// v[l >> (6 - log2 N)], complete in every lane of its group of 64 / N.
template <int M, int N, int CAP>
__device__ __forceinline__ void halve(float (&w)[CAP], int lane) {
    const bool up = (lane & M) != 0;
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
        const float keep = up ? w[i + N / 2] : w[i];
        const float send = up ? w[i] : w[i + N / 2];
        w[i] = keep + dev::xor_lane<M>(send);
    }
}

template <int N, int CAP>
__device__ __forceinline__ float reduce_scatter(float (&w)[CAP], int lane) {
    static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16, "one to sixteen sums");
    // The first log2 N exchanges use masks 32, 16, ... in turn.
    constexpr int L = N == 16 ? 4 : N == 8 ? 3 : N == 4 ? 2 : N == 2 ? 1 : 0;
    if constexpr (L >= 4) halve<32, 16>(w, lane);
    if constexpr (L >= 3) halve<(32 >> (L - 3)), 8>(w, lane);
    if constexpr (L >= 2) halve<(32 >> (L - 2)), 4>(w, lane);
    if constexpr (L >= 1) halve<(32 >> (L - 1)), 2>(w, lane);
    float v = w[0];
    if constexpr (L < 1) v += dev::xor_lane<32>(v);
    if constexpr (L < 2) v += dev::xor_lane<16>(v);
    if constexpr (L < 3) v += dev::xor_lane<8>(v);
    if constexpr (L < 4) v += dev::xor_lane<4>(v);
    v += dev::xor_lane<2>(v);
    return v + dev::xor_lane<1>(v);
}

constexpr int log2_tokens(int tok) { return tok == 4 ? 2 : tok == 2 ? 1 : 0; }

// Stores a unit's outputs from its reduced sums: acc[0] the (gate) row's
// TOK token sums, acc[1] the up row's with pairs. Without pairs lane l holds
// token l >> (6 - log2 TOK)'s sum; with pairs the gate sums come first, so a
// gate lane's up sum is 32 lanes away.
template <int TOK>
__device__ __forceinline__ void store_unit(const DenseArgs &a, float (&acc)[2][TOK], uint32_t o, uint32_t first,
                                           int lane) {
    constexpr int LT = log2_tokens(TOK);
    if (a.pairs) {
        float w[2 * TOK];
#pragma unroll
        for (int t = 0; t < TOK; ++t) {
            w[t] = acc[0][t];
            w[TOK + t] = acc[1][t];
        }
        const float g = reduce_scatter<2 * TOK>(w, lane);
        const float u = dev::xor_lane<32>(g);
        const uint32_t t = (uint32_t)lane >> (5 - LT);
        if ((lane & ((32 >> LT) - 1)) == 0 && lane < 32 && first + t < a.tokens)
            a.out[(size_t)(first + t) * (a.rows / 2) + o] = __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, expf(-g))), u);
    } else {
        float w[TOK];
#pragma unroll
        for (int t = 0; t < TOK; ++t) w[t] = acc[0][t];
        const float y = reduce_scatter<TOK>(w, lane);
        const uint32_t t = (uint32_t)lane >> (6 - LT);
        if ((lane & ((64 >> LT) - 1)) == 0 && first + t < a.tokens) {
            const size_t at = (size_t)(first + t) * a.rows + o;
            a.out[at] = a.residual ? a.residual[at] + y : y;
        }
    }
}

// A wavefront's work in 16-byte slices: units (one output: a row, or with
// pairs its gate and up rows) in grid-stride order, each row in chunks of
// four slices per lane (lane l takes slices l, l + 64, l + 128, l + 192 of
// the chunk's 256). Chunk j of the sequence is (unit, row r, chunk c).
struct ChunkPos {
    uint32_t unit, r, c;
};

__device__ __forceinline__ void chunk_next(ChunkPos &p, uint32_t rows_per_unit, uint32_t cpr) {
    if (++p.c == cpr) {
        p.c = 0;
        if (++p.r == rows_per_unit) {
            p.r = 0;
            ++p.unit;
        }
    }
}

// The chunk's four 16-byte loads (slices past the row load its last slice
// again: not used).
template <bool Half>
__device__ __forceinline__ void load_chunk(const DenseArgs &a, const ChunkPos &p, uint32_t wave, uint32_t nwaves,
                                           uint32_t rows_per_unit, uint32_t slices, int lane, u32x4 (&v)[4]) {
    const uint32_t o = wave + p.unit * nwaves;
    const uint32_t row = rows_per_unit * o + p.r;
    const u32x4 *src = reinterpret_cast<const u32x4 *>(a.w) + (size_t)row * slices;
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = __builtin_nontemporal_load(src + min(p.c * 256u + lane + 64u * u, slices - 1));
}

template <bool Half, bool Norm, int TOK>
__global__ __launch_bounds__(256) void gemv_dense_kernel(const DenseArgs a) {
    extern __shared__ float4 lds4[];
    float *xs = reinterpret_cast<float *>(lds4);  // TOK x cols activations, then TOK x 4 partial sums
    const int tid = threadIdx.x, lane = tid & 63;
    const uint32_t cols = a.cols;
    const uint32_t first = blockIdx.y * TOK;
    constexpr uint32_t kPer = Half ? 8 : 4;
    const bool sliced = cols % kPer == 0 && ((uintptr_t)a.w & 15u) == 0;
    const uint32_t wave = blockIdx.x * 4 + (tid >> 6), nwaves = gridDim.x * 4;
    const uint32_t rows_per_unit = a.pairs ? 2u : 1u;
    const uint32_t outputs = a.rows / rows_per_unit;
    const uint32_t units = wave < outputs ? (outputs - wave + nwaves - 1) / nwaves : 0;
    const uint32_t slices = cols / kPer;
    const uint32_t cpr = (slices + 255) / 256;  // chunks per row
    const uint32_t total = sliced ? units * rows_per_unit * cpr : 0;
    // Token groups past the last token repeat it (their sums are not stored).
    uint32_t token[TOK];
#pragma unroll
    for (int t = 0; t < TOK; ++t) token[t] = min(first + t, a.tokens - 1);
    // f16 slices: value j of slice c at c * 4 + (j & 3), in the second plane
    // (cols / 2 further on) for j >= 4, so each lane's LDS reads are whole
    // 16-byte words.
    const bool split = Half && sliced;
    auto slot = [&](uint32_t k) { return split ? ((k & 4u) ? cols / 2 : 0u) + (k >> 3) * 4 + (k & 3u) : k; };
    // The prologue's loads in the order they are needed: the thread's first
    // kBatch activations of each token (and their RMSNorm weights), then the
    // first chunk's weights, so that using the activations waits only for
    // their own loads (loads complete in issue order) while the weights stay
    // in flight. Columns past the row load its last column (not stored).
    constexpr int kBatch = 8;
    constexpr uint32_t kSpan = 256u * kBatch;  // columns per batch of the workgroup
    // One token's first batch stays in registers until RMSNorm scales it;
    // with more tokens it goes to LDS as it is (fewer registers held).
    constexpr bool kKeep = TOK == 1;
    float v[TOK][kBatch], nw[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
        const uint32_t k = min(tid + 256u * i, cols - 1);
#pragma unroll
        for (int t = 0; t < TOK; ++t) v[t][i] = a.x[(size_t)token[t] * cols + k];
        if constexpr (Norm) nw[i] = a.norm[k];
    }
    ChunkPos pos{0, 0, 0};
    u32x4 cur[4];
    if (total) load_chunk<Half>(a, pos, wave, nwaves, rows_per_unit, slices, lane, cur);
    float ss[TOK];
#pragma unroll
    for (int t = 0; t < TOK; ++t) {
        ss[t] = 0.0f;
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            const uint32_t k = tid + 256u * i;
            if (k < cols) {
                if constexpr (Norm) ss[t] = __fadd_rn(ss[t], __fmul_rn(v[t][i], v[t][i]));
                if constexpr (!Norm || !kKeep) xs[(size_t)t * cols + slot(k)] = v[t][i];
            }
        }
    }
    // Rows wider than one batch: the rest in batches of kBatch loads in
    // flight together, stored as they are (RMSNorm scales them below).
    for (uint32_t base = kSpan; base < cols; base += kSpan) {
        float r[TOK][kBatch];
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            const uint32_t k = min(base + tid + 256u * i, cols - 1);
#pragma unroll
            for (int t = 0; t < TOK; ++t) r[t][i] = a.x[(size_t)token[t] * cols + k];
        }
#pragma unroll
        for (int t = 0; t < TOK; ++t)
#pragma unroll
            for (int i = 0; i < kBatch; ++i) {
                const uint32_t k = base + tid + 256u * i;
                if (k < cols) {
                    if constexpr (Norm) ss[t] = __fadd_rn(ss[t], __fmul_rn(r[t][i], r[t][i]));
                    xs[(size_t)t * cols + slot(k)] = r[t][i];
                }
            }
    }
    if constexpr (Norm) {
        // math.zig:118-130: x * (1 / sqrt(mean(x^2) + eps)) * w, the sum of
        // squares reduced over the block (threads, then the four waves in
        // order).
        float *partial = xs + (size_t)TOK * cols;
#pragma unroll
        for (int t = 0; t < TOK; ++t) {
            const float w = dev::wave_sum(ss[t]);
            if (lane == 0) partial[t * 4 + (tid >> 6)] = w;
        }
        __syncthreads();
        float inv[TOK];
#pragma unroll
        for (int t = 0; t < TOK; ++t) {
            const float *p = partial + t * 4;
            const float sum = ((p[0] + p[1]) + p[2]) + p[3];
            inv[t] = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(sum, (float)cols), a.eps)));
        }
        // The first batch from registers (or LDS), the rest from LDS with
        // their weights loaded a batch at a time.
#pragma unroll
        for (int t = 0; t < TOK; ++t)
#pragma unroll
            for (int i = 0; i < kBatch; ++i) {
                const uint32_t k = tid + 256u * i;
                if (k < cols) {
                    float &x = xs[(size_t)t * cols + slot(k)];
                    x = __fmul_rn(__fmul_rn(kKeep ? v[t][i] : x, inv[t]), nw[i]);
                }
            }
        for (uint32_t base = kSpan; base < cols; base += kSpan) {
            float w[kBatch];
#pragma unroll
            for (int i = 0; i < kBatch; ++i) w[i] = a.norm[min(base + tid + 256u * i, cols - 1)];
#pragma unroll
            for (int t = 0; t < TOK; ++t)
#pragma unroll
                for (int i = 0; i < kBatch; ++i) {
                    const uint32_t k = base + tid + 256u * i;
                    if (k < cols) {
                        float &x = xs[(size_t)t * cols + slot(k)];
                        x = __fmul_rn(__fmul_rn(x, inv[t]), w[i]);
                    }
                }
        }
    }
    __syncthreads();
    float acc[2][TOK];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int t = 0; t < TOK; ++t) acc[r][t] = 0.0f;
    if (sliced) {
        const uint32_t hi_off = Half ? cols / 2 : 0;
        ChunkPos next = pos;
        for (uint32_t j = 0; j < total; ++j) {
            // The next chunk's loads go out before this one is multiplied
            // (the last chunk loads itself again).
            if (j + 1 < total) chunk_next(next, rows_per_unit, cpr);
            u32x4 nxt[4];
            load_chunk<Half>(a, next, wave, nwaves, rows_per_unit, slices, lane, nxt);
            float part[TOK];
#pragma unroll
            for (int t = 0; t < TOK; ++t) part[t] = 0.0f;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t c = pos.c * 256u + lane + 64u * u;
                if (c < slices) {
#pragma unroll
                    for (int t = 0; t < TOK; ++t) {
                        const float *xt = xs + (size_t)t * cols + c * 4;
                        const float4 lo = *reinterpret_cast<const float4 *>(xt);
                        const float4 hi = Half ? *reinterpret_cast<const float4 *>(xt + hi_off) : lo;
                        part[t] += slice_dot<Half>(cur[u], lo, hi);
                    }
                }
            }
            if (pos.r == 0) {
#pragma unroll
                for (int t = 0; t < TOK; ++t) acc[0][t] += part[t];
            } else {
#pragma unroll
                for (int t = 0; t < TOK; ++t) acc[1][t] += part[t];
            }
            if (pos.c + 1 == cpr && pos.r + 1 == rows_per_unit) {
                store_unit<TOK>(a, acc, wave + pos.unit * nwaves, first, lane);
#pragma unroll
                for (int r = 0; r < 2; ++r)
#pragma unroll
                    for (int t = 0; t < TOK; ++t) acc[r][t] = 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) cur[u] = nxt[u];
            pos = next;
        }
    } else {
        // Rows that are not whole 16-byte slices: element by element.
        const size_t elem = Half ? 2 : 4;
        for (uint32_t i = 0; i < units; ++i) {
            const uint32_t o = wave + i * nwaves;
            for (uint32_t r = 0; r < rows_per_unit; ++r) {
                const uint8_t *base = a.w + (size_t)(rows_per_unit * o + r) * cols * elem;
                float part[TOK];
#pragma unroll
                for (int t = 0; t < TOK; ++t) part[t] = 0.0f;
                for (uint32_t k = lane; k < cols; k += 64) {
                    const float w = dense_weight<Half>(base, k);
#pragma unroll
                    for (int t = 0; t < TOK; ++t) part[t] = fmaf(w, xs[(size_t)t * cols + k], part[t]);
                }
                if (r == 0) {
#pragma unroll
                    for (int t = 0; t < TOK; ++t) acc[0][t] = part[t];
                } else {
#pragma unroll
                    for (int t = 0; t < TOK; ++t) acc[1][t] = part[t];
                }
            }
            store_unit<TOK>(a, acc, o, first, lane);
        }
    }
}

// ---- Sixteen tokens at a time on the matrix cores ----
//
// A workgroup computes a 16-row x 16-token tile with v_mfma_f32_16x16x4_f32:
// lane l supplies A[m = l % 16][k = l / 16] (token m's activation) and
// B[k = l / 16][n = l % 16] (row n's weight), and holds C[4 (l / 16) + i]
// [l % 16] in value i. Each K-step covers four lane groups of one 16-byte
// weight load each (8 f16 or 4 f32 columns): MFMA e of the step multiplies
// column step + 8 g + e (f16; 4 g + e for f32) for lane group g. The four
// wavefronts split the K-steps into quarters and their tiles are summed in
// order through LDS, so the result does not depend on timing. RMSNorm's
// weights multiply the activations as they are read; the 1 / rms factor of
// each token, from the sums of squares the wavefronts gather on the way,
// scales the tile once at the end (a rounding apart from the reference's
// (x * inv) * w, like the int8 batch GEMV's RMSNorm form).
typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int kMmaDepth = 8;  // K-steps of loads in flight per wavefront

template <bool Half, bool Norm>
__global__ __launch_bounds__(256) void gemm_dense_kernel(const DenseArgs a) {
    constexpr uint32_t kPer = Half ? 8 : 4;   // values per 16-byte weight load
    constexpr uint32_t kCols = 4 * kPer;      // columns per K-step
    constexpr int kX = kPer / 4;              // float4 activation loads per lane per step
    extern __shared__ float4 lds_dyn[];
    float *lds_norm = reinterpret_cast<float *>(lds_dyn);  // RMSNorm weights, cols values
    __shared__ float part[4][16][17];
    __shared__ float ssp[4][16];
    __shared__ float sums[16][17];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, g = lane >> 4;
    const uint32_t row0 = blockIdx.x * 16, tok0 = blockIdx.y * 16;
    const uint32_t row = min(row0 + li, a.rows - 1);    // B operand row (rows past the matrix repeat the last)
    const uint32_t tok = min(tok0 + li, a.tokens - 1);  // A operand token (likewise)
    const uint32_t steps = a.cols / kCols;
    const uint32_t s_begin = wave * steps / 4, n_steps = (wave + 1) * steps / 4 - s_begin;
    const u32x4 *wrow = reinterpret_cast<const u32x4 *>(a.w) + (size_t)row * (a.cols / kPer);
    const float4 *xrow = reinterpret_cast<const float4 *>(a.x + (size_t)tok * a.cols);
    u32x4 wb[kMmaDepth];
    float4 xa[kMmaDepth][kX];
    // Step s of this wavefront's quarter into slot `slot` (steps past the
    // quarter load its last step again: not used).
    auto issue = [&](uint32_t s, int slot) {
        const uint32_t col = (s_begin + min(s, n_steps - 1)) * kCols + g * kPer;
        wb[slot] = __builtin_nontemporal_load(wrow + col / kPer);
#pragma unroll
        for (int h = 0; h < kX; ++h) xa[slot][h] = xrow[col / 4 + h];
    };
#pragma unroll
    for (int i = 0; i < kMmaDepth; ++i) issue(i, i);
    if constexpr (Norm) {
        // The norm weights into LDS: requested after the first steps'
        // weights, so waiting for them leaves nothing of those in flight
        // that was not already due.
        for (uint32_t k = 4 * tid; k < a.cols; k += 4 * 256 * 8) {
            float4 v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = reinterpret_cast<const float4 *>(a.norm)[min(k + 1024u * j, a.cols - 4) / 4];
#pragma unroll
            for (int j = 0; j < 8; ++j) reinterpret_cast<float4 *>(lds_norm)[min(k + 1024u * j, a.cols - 4) / 4] = v[j];
        }
        __syncthreads();
    }
    v4f c0 = {0.0f, 0.0f, 0.0f, 0.0f}, c1 = {0.0f, 0.0f, 0.0f, 0.0f};
    float ss = 0.0f;
    for (uint32_t base = 0; base < n_steps; base += kMmaDepth) {
#pragma unroll
        for (int i = 0; i < kMmaDepth; ++i) {
            if (base + i < n_steps) {
                const uint32_t col = (s_begin + base + i) * kCols + g * kPer;
                const u32x4 w = wb[i];
                const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                for (int e = 0; e < (int)kPer; ++e) {
                    const float4 xv4 = xa[i][e / 4];
                    float xv = (e & 3) == 0 ? xv4.x : (e & 3) == 1 ? xv4.y : (e & 3) == 2 ? xv4.z : xv4.w;
                    if constexpr (Norm) {
                        ss = __fadd_rn(ss, __fmul_rn(xv, xv));
                        xv = __fmul_rn(xv, lds_norm[col + e]);
                    }
                    const float wv = Half ? dev::f16_bits_to_f32((uint16_t)(words[e / 2] >> (16 * (e & 1))))
                                          : __uint_as_float(words[e]);
                    if (e & 1) c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(xv, wv, c1, 0, 0, 0);
                    else c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(xv, wv, c0, 0, 0, 0);
                }
            }
            issue(base + i + kMmaDepth, i);
        }
    }
    const v4f c = c0 + c1;
#pragma unroll
    for (int i = 0; i < 4; ++i) part[wave][4 * g + i][li] = c[i];
    if constexpr (Norm) {
        // Lanes li, li + 16, li + 32, li + 48 hold token li's squares.
        ss += dev::xor_lane<16>(ss);
        ss += dev::xor_lane<32>(ss);
        if (g == 0) ssp[wave][li] = ss;
    }
    __syncthreads();
    const int m = tid >> 4, n = tid & 15;  // this thread's token and row in the tile
    float y = ((part[0][m][n] + part[1][m][n]) + part[2][m][n]) + part[3][m][n];
    if constexpr (Norm) {
        const float sum = ((ssp[0][m] + ssp[1][m]) + ssp[2][m]) + ssp[3][m];
        y = __fmul_rn(y, __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(sum, (float)a.cols), a.eps))));
    }
    const uint32_t t_out = tok0 + m, r_out = row0 + n;
    if (a.pairs) {
        sums[m][n] = y;
        __syncthreads();
        if ((n & 1) == 0 && t_out < a.tokens && r_out < a.rows) {
            const float gt = sums[m][n], up = sums[m][n + 1];
            a.out[(size_t)t_out * (a.rows / 2) + r_out / 2] = __fmul_rn(__fdiv_rn(gt, __fadd_rn(1.0f, expf(-gt))), up);
        }
    } else if (t_out < a.tokens && r_out < a.rows) {
        const size_t at = (size_t)t_out * a.rows + r_out;
        a.out[at] = a.residual ? a.residual[at] + y : y;
    }
}

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f2 __attribute__((ext_vector_type(2)));

// One K-step of a lane's activations (16 of its token's 64 in the step) as
// f16 operands, hi + lo = x * s to within 2^-22 of the step's largest
// magnitude, and the 1 / s that undoes the scale. s = 2^(14 - E) for the
// largest magnitude's exponent E over the token's 64 values (the lanes l,
// l ^ 16, l ^ 32, l ^ 48 hold them), so the scaled values stay below 2^15,
// inside the f16 range, and keep their f32 precision in the pair: hi is x * s
// rounded to f16, lo the exact f32 remainder rounded to f16. Exponents are
// clamped to [2^-112, inf], so s and 1 / s are normal powers of two and the
// scaling is exact. A NaN or inf in the step carries through to the sums: an
// inf is its own hi (lo 0, where the remainder would be NaN), a NaN makes
// both NaN.
__device__ __forceinline__ float split_step(const float (&xv)[16], h8 (&hi)[2], h8 (&lo)[2]) {
    float m[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
        m[q] = fmaxf(fmaxf(fabsf(xv[4 * q]), fabsf(xv[4 * q + 1])), fmaxf(fabsf(xv[4 * q + 2]), fabsf(xv[4 * q + 3])));
    float mx = fmaxf(fmaxf(m[0], m[1]), fmaxf(m[2], m[3]));
    mx = fmaxf(mx, dev::xor_lane<16>(mx));
    mx = fmaxf(mx, dev::xor_lane<32>(mx));
    const uint32_t e = max(__float_as_uint(mx) & 0x7F800000u, 15u << 23);
    const bool inf = e == 0x7F800000u;
    const float s = __uint_as_float((268u << 23) - e);  // 2^(141 - biased exponent)
#pragma unroll
    for (int j = 0; j < 16; j += 2) {
        const f2 v = {__fmul_rn(xv[j], s), __fmul_rn(xv[j + 1], s)};
        const h2 h = __builtin_convertvector(v, h2);
        const h2 l = __builtin_convertvector(v - __builtin_convertvector(h, f2), h2);
        hi[j / 8][j % 8] = h.x;
        hi[j / 8][j % 8 + 1] = h.y;
        lo[j / 8][j % 8] = inf ? (_Float16)0.0f : l.x;
        lo[j / 8][j % 8 + 1] = inf ? (_Float16)0.0f : l.y;
    }
    return __uint_as_float(e - (14u << 23));  // 1 / s
}

// f16 weights on the f16 matrix cores (v_mfma_f32_16x16x32_f16), from eight
// tokens: the products w * hi and w * lo are exact in f32, so the sums carry
// f32 precision. A workgroup holds 16 * R rows x 16 tokens; its W wavefronts
// split K in steps of 64 values and add their tiles through LDS in a fixed
// order. Per step a lane holds, for each row tile, 16 weights of row l % 16:
// values 8 (l / 16) .. + 7 of each half of the step, the A operands of two
// MFMAs (each load covers 64 contiguous bytes of 16 rows). The activations
// are loaded whole rows at a time (each load covers 256 contiguous bytes of
// four tokens), passed through a per-wavefront LDS tile, and read back as
// the same 16 positions of token l % 16 (the B operands), so a lane's
// accumulators are rows 4 (l / 16) + i of its own token and take that
// token's 1 / s. Loads go through buffer resources bounded by the tile:
// rows and tokens past the matrix or batch, and the steps past a
// wavefront's range that keep the pipeline's shape, read zeros and touch no
// memory. D steps of loads are in flight per wavefront. With RMSNorm the
// norm weights sit in LDS, each activation is scaled as it is read, and the
// token's inverse RMS multiplies the sums at the end.
template <bool Norm, int R, int W, int D>
__global__ __launch_bounds__(64 * W) void gemm_f16_kernel(const DenseArgs a) {
    extern __shared__ float4 lds_dyn[];      // RMSNorm weights, cols values
    __shared__ float4 xtile[W][16 * 17];     // per wavefront: 16 tokens x 64 values (+ 4 of padding)
    __shared__ float part[W][16 * R][17];
    __shared__ float ssp[W][16];
    constexpr uint32_t kFar = 0x7FFFFF00u;  // an offset past every tile
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, g = lane >> 4;
    const uint32_t row0 = blockIdx.x * (16u * R), tok0 = blockIdx.y * 16;
    const uint32_t nrows = min(16u * R, a.rows - row0), ntok = min(16u, a.tokens - tok0);
    const uint32_t steps = a.cols / 64;
    const uint32_t s_begin = wave * steps / W, n_steps = (wave + 1) * steps / W - s_begin;
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(a.w) + (size_t)row0 * a.cols * 2, (short)0, (int)(nrows * a.cols * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(a.x) + (size_t)tok0 * a.cols, (short)0, (int)(ntok * a.cols * 4), 0x00020000);
    const uint32_t w_lane = (uint32_t)li * a.cols * 2 + 16u * g + 128u * s_begin;
    const uint32_t x_lane = (uint32_t)g * a.cols * 4 + 16u * li + 256u * s_begin;
    u32x4 wb[D][R][2];
    u32x4 xa[D][4];
    // Step s of this wavefront's range into slot `slot` (past the range: no
    // memory is read), the same loads every iteration, so each step waits
    // only for its own.
    auto issue = [&](uint32_t s, int slot) {
        const bool valid = s < n_steps;
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                wb[slot][r][h] = __builtin_amdgcn_raw_buffer_load_b128(
                    wres, valid ? w_lane + 16u * r * a.cols * 2 + 128u * s + 64u * h : kFar, 0, 2 /* nt */);
#pragma unroll
        for (int b = 0; b < 4; ++b)
            xa[slot][b] = __builtin_amdgcn_raw_buffer_load_b128(
                xres, valid ? x_lane + 4u * b * a.cols * 4 + 256u * s : kFar, 0, 0);
    };
#pragma unroll
    for (int i = 0; i < D; ++i) {
        issue(i, i);
        __builtin_amdgcn_sched_barrier(0);  // slots in order: step 0's loads first
    }
    if constexpr (Norm) {
        // The RMSNorm weights into LDS, requested after the first steps'
        // loads: waiting for them coincides with those. Each batch's stores
        // are unconditional (past the row, the last four values again, to
        // their own place), so its loads go out together (2048 values per
        // pass, J loads per thread: more would not stay in registers beside
        // the slots in flight).
        constexpr int J = W >= 8 ? 1 : 8 / W;
        const float4 *norm4 = reinterpret_cast<const float4 *>(a.norm);
        for (uint32_t k = 4 * tid; k < a.cols; k += 256u * W * J) {
            float4 v[J];
#pragma unroll
            for (int j = 0; j < J; ++j) v[j] = norm4[min(k + 256u * W * j, a.cols - 4) / 4];
            __builtin_amdgcn_sched_barrier(0);  // all J loads before the first store
#pragma unroll
            for (int j = 0; j < J; ++j) lds_dyn[min(k + 256u * W * j, a.cols - 4) / 4] = v[j];
        }
        __syncthreads();
    }
    float4 *xt = xtile[wave];
    v4f acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    float ss = 0.0f;
    // Every iteration runs the same straight-line code; a step past the
    // range (zeros) leaves the sums unchanged.
    for (uint32_t base = 0; base < n_steps; base += D) {
#pragma unroll
        for (int i = 0; i < D; ++i) {
            const bool valid = base + i < n_steps;
            // Tokens g + 4 b, 4 values at 4 li, into the tile; read back
            // token li's values at 8 g and 32 + 8 g.
#pragma unroll
            for (int b = 0; b < 4; ++b) xt[(g + 4 * b) * 17 + li] = __builtin_bit_cast(float4, xa[i][b]);
            float xv[16];
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const float4 v = xt[li * 17 + 8 * (h >> 1) + 2 * g + (h & 1)];
                xv[4 * h] = v.x;
                xv[4 * h + 1] = v.y;
                xv[4 * h + 2] = v.z;
                xv[4 * h + 3] = v.w;
            }
            if constexpr (Norm) {
                const uint32_t st = s_begin + min(base + i, n_steps - 1);
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    const float4 n4 = lds_dyn[st * 16 + 8 * (h >> 1) + 2 * g + (h & 1)];
                    const float nv[4] = {n4.x, n4.y, n4.z, n4.w};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const float sq = __fadd_rn(ss, __fmul_rn(xv[4 * h + j], xv[4 * h + j]));
                        ss = valid ? sq : ss;
                        xv[4 * h + j] = __fmul_rn(xv[4 * h + j], nv[j]);
                    }
                }
            }
            h8 hi[2], lo[2];
            const float inv = split_step(xv, hi, lo);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const h8 w0 = __builtin_bit_cast(h8, wb[i][r][0]), w1 = __builtin_bit_cast(h8, wb[i][r][1]);
                v4f t = __builtin_amdgcn_mfma_f32_16x16x32_f16(w0, hi[0], v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                t = __builtin_amdgcn_mfma_f32_16x16x32_f16(w1, hi[1], t, 0, 0, 0);
                t = __builtin_amdgcn_mfma_f32_16x16x32_f16(w0, lo[0], t, 0, 0, 0);
                t = __builtin_amdgcn_mfma_f32_16x16x32_f16(w1, lo[1], t, 0, 0, 0);
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const float sum = __fmaf_rn(t[c], inv, acc[r][c]);
                    acc[r][c] = valid ? sum : acc[r][c];
                }
            }
            issue(base + i + D, i);
            // The next step's work stays after this step's loads are issued
            // (moved up, it would wait for the next slot's loads early).
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) part[wave][16 * r + 4 * g + c][li] = acc[r][c];
    if constexpr (Norm) {
        // Lanes li, li + 16, li + 32, li + 48 hold token li's squares.
        ss += dev::xor_lane<16>(ss);
        ss += dev::xor_lane<32>(ss);
        if (g == 0) ssp[wave][li] = ss;
    }
    __syncthreads();
    auto total = [&](int n, int m) {
        float y = part[0][n][m];
#pragma unroll
        for (int v = 1; v < W; ++v) y += part[v][n][m];
        if constexpr (Norm) {
            float sum = ssp[0][m];
#pragma unroll
            for (int v = 1; v < W; ++v) sum += ssp[v][m];
            y = __fmul_rn(y, __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(sum, (float)a.cols), a.eps))));
        }
        return y;
    };
    if (a.pairs) {
        // 8 R gate / up pairs x 16 tokens.
        for (int idx = tid; idx < 128 * R; idx += 64 * W) {
            const int m = idx / (8 * R), p = idx % (8 * R);
            const uint32_t t_out = tok0 + m, r_out = row0 + 2 * p;
            if (t_out < a.tokens && r_out < a.rows) {
                const float gt = total(2 * p, m), up = total(2 * p + 1, m);
                a.out[(size_t)t_out * (a.rows / 2) + r_out / 2] = __fmul_rn(__fdiv_rn(gt, __fadd_rn(1.0f, expf(-gt))), up);
            }
        }
    } else {
        for (int idx = tid; idx < 256 * R; idx += 64 * W) {
            const int m = idx / (16 * R), n = idx % (16 * R);
            const uint32_t t_out = tok0 + m, r_out = row0 + n;
            if (t_out < a.tokens && r_out < a.rows) {
                const float y = total(n, m);
                const size_t at = (size_t)t_out * a.rows + r_out;
                a.out[at] = a.residual ? a.residual[at] + y : y;
            }
        }
    }
}

// f16 weights, many rows or tokens: the same split activations, with each
// of the workgroup's W wavefronts on its own R row tiles (all of K) and T
// token tiles sharing every weight load. The activations are loaded, scaled
// and split once per workgroup, C steps at a time, into LDS in the MFMA
// operand layout (double buffered, one barrier per chunk), so the address
// unit moves each activation once per 16 R W rows. A unit of staging is one
// step of one token tile: 128 threads, each with 8 consecutive values of
// one token (two 16-byte loads; the token's 64 values are 8 neighbouring
// lanes, whose maximum three DPP exchanges give), writing one 16-byte hi and
// one lo operand lane. Operand lane 16 g + li of half h sits at position
// 16 g + ((li + 2 g + 8 h) mod 16) of its 64: a wavefront reads an operand
// as 64 distinct 16-byte words, and the writers of one pass hit 16
// distinct bank groups. The weights stream C steps ahead through a bounded
// buffer resource (rows past the matrix and steps past the row read zeros,
// no memory). A lane's accumulators are rows 4 (l / 16) + i of its tile for
// token l % 16, so the epilogue needs no cross-wavefront sum: residual,
// siluMul of gate / up pairs (rows 2p, 2p + 1 sit in the same lane), or
// RMSNorm's inverse RMS per token.
template <bool Norm, int R, int T, int W>
__global__ __launch_bounds__(64 * W) void gemm_f16_rows_kernel(const DenseArgs a) {
    constexpr int C = 2;                      // steps per chunk, and steps of weight loads in flight
    constexpr int kUnits = C * T;             // staging units per chunk: [tile][step]
    constexpr int kGroups = W / 2;            // 128-thread staging groups
    constexpr int NU = kUnits / kGroups;      // units per thread per chunk
    static_assert(kUnits % kGroups == 0, "whole units per staging group");
    constexpr int kOps = kUnits * 4 * 64;     // u32x4 operands per buffer: [step][tile][half][hi/lo][64]
    constexpr int kInv = kUnits * 16;         // 1 / s per buffer: [step][tile][token]
    constexpr uint32_t kFar = 0x7FFFFF00u;
    extern __shared__ float4 lds_dyn[];       // RMSNorm weights (cols values), then the two buffers
    __shared__ float sspart[kGroups][T][16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, g = lane >> 4;
    const uint32_t rows_wg = 16u * R * W;
    const uint32_t row0 = blockIdx.x * rows_wg, tok0 = blockIdx.y * (16u * T);
    const uint32_t nrows = min(rows_wg, a.rows - row0), ntok = min(16u * T, a.tokens - tok0);
    const uint32_t steps = a.cols / 64, chunks = (steps + C - 1) / C;
    u32x4 *ops = reinterpret_cast<u32x4 *>(lds_dyn + (Norm ? a.cols / 4 : 0));
    float *invs = reinterpret_cast<float *>(ops + 2 * kOps);
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(a.w) + (size_t)row0 * a.cols * 2, (short)0, (int)(nrows * a.cols * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(a.x) + (size_t)tok0 * a.cols, (short)0, (int)(ntok * a.cols * 4), 0x00020000);
    const uint32_t w_lane = ((uint32_t)wave * 16u * R + li) * a.cols * 2 + 16u * g;
    // Staging thread: group gamma, token tt of the unit's tile, values 8 q8 .. + 7 of its step.
    const int gamma = tid >> 7, tt = (tid >> 3) & 15, q8 = tid & 7;
    const int hf = q8 >> 2, gq = q8 & 3;
    const int pos = 16 * gq + ((tt + 2 * gq + 8 * hf) & 15);  // operand word of this thread
    u32x4 wb[C][R][2];
    auto issue_w = [&](uint32_t s, int slot) {
        const bool valid = s < steps;
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                wb[slot][r][h] = __builtin_amdgcn_raw_buffer_load_b128(
                    wres, valid ? w_lane + 16u * r * a.cols * 2 + 128u * s + 64u * h : kFar, 0, 2 /* nt */);
        asm volatile("" ::: "memory");
    };
    u32x4 xr[NU][2];
    // Unit u = gamma + kGroups j of a chunk: tile u / C, step u % C.
    auto issue_x = [&](uint32_t chunk) {
#pragma unroll
        for (int j = 0; j < NU; ++j) {
            const int u = gamma + kGroups * j, t = u / C, i = u % C;
            const uint32_t s = chunk * C + i;
            const uint32_t off = ((16u * t + tt) * a.cols + 64u * s + 8u * q8) * 4;
#pragma unroll
            for (int h = 0; h < 2; ++h)
                xr[j][h] = __builtin_amdgcn_raw_buffer_load_b128(xres, s < steps ? off + 16u * h : kFar, 0, 0);
        }
        asm volatile("" ::: "memory");
    };
    float ss[T];
#pragma unroll
    for (int t = 0; t < T; ++t) ss[t] = 0.0f;
    auto stage_x = [&](uint32_t chunk, int buf) {
#pragma unroll
        for (int j = 0; j < NU; ++j) {
            const int u = gamma + kGroups * j, t = u / C, i = u % C;
            const uint32_t s = min(chunk * C + i, steps - 1);
            const float4 x0 = __builtin_bit_cast(float4, xr[j][0]), x1 = __builtin_bit_cast(float4, xr[j][1]);
            float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            if constexpr (Norm) {
                // (Steps past the row read zeros and add nothing.)
                const float4 n0 = lds_dyn[s * 16 + 2 * q8], n1 = lds_dyn[s * 16 + 2 * q8 + 1];
                const float nv[8] = {n0.x, n0.y, n0.z, n0.w, n1.x, n1.y, n1.z, n1.w};
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    ss[t] = __fadd_rn(ss[t], __fmul_rn(v[k], v[k]));
                    v[k] = __fmul_rn(v[k], nv[k]);
                }
            }
            float mx = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; ++k) mx = fmaxf(mx, fabsf(v[k]));
            mx = fmaxf(mx, dev::xor_lane<1>(mx));
            mx = fmaxf(mx, dev::xor_lane<2>(mx));
            mx = fmaxf(mx, dev::xor_lane<4>(mx));
            const uint32_t e = max(__float_as_uint(mx) & 0x7F800000u, 15u << 23);
            const bool inf = e == 0x7F800000u;
            const float sc = __uint_as_float((268u << 23) - e);
            u32x4 hw, lw;
#pragma unroll
            for (int k = 0; k < 8; k += 2) {
                const f2 fv = {__fmul_rn(v[k], sc), __fmul_rn(v[k + 1], sc)};
                const h2 h = __builtin_convertvector(fv, h2);
                h2 l = __builtin_convertvector(fv - __builtin_convertvector(h, f2), h2);
                if (inf) l = h2{(_Float16)0.0f, (_Float16)0.0f};
                hw[k / 2] = __builtin_bit_cast(uint32_t, h);
                lw[k / 2] = __builtin_bit_cast(uint32_t, l);
            }
            u32x4 *dst = ops + buf * kOps + ((i * T + t) * 2 + hf) * 2 * 64 + pos;
            dst[0] = hw;
            dst[64] = lw;
            if (q8 == 0) invs[buf * kInv + (i * T + t) * 16 + tt] = __uint_as_float(e - (14u << 23));
        }
    };
#pragma unroll
    for (int i = 0; i < C; ++i) {
        issue_w(i, i);
        __builtin_amdgcn_sched_barrier(0);
    }
    issue_x(0);
    if constexpr (Norm) {
        // The RMSNorm weights into LDS (two loads per thread per pass,
        // stored unconditionally: past the row, the last four again).
        const float4 *norm4 = reinterpret_cast<const float4 *>(a.norm);
        for (uint32_t k = 4 * tid; k < a.cols; k += 512u * W) {
            const float4 v0 = norm4[min(k, a.cols - 4) / 4], v1 = norm4[min(k + 256u * W, a.cols - 4) / 4];
            __builtin_amdgcn_sched_barrier(0);
            lds_dyn[min(k, a.cols - 4) / 4] = v0;
            lds_dyn[min(k + 256u * W, a.cols - 4) / 4] = v1;
        }
        __syncthreads();
    }
    stage_x(0, 0);
    __syncthreads();
    v4f acc[R][T];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[r][t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    // Operand lane `lane` of a 64-word operand.
    const int rpos = 16 * g + ((li + 2 * g) & 15);
    for (uint32_t c = 0; c < chunks; ++c) {
        const int buf = c & 1;
        if (c + 1 < chunks) issue_x(c + 1);
#pragma unroll
        for (int i = 0; i < C; ++i) {
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const u32x4 *op = ops + buf * kOps + (i * T + t) * 4 * 64;
                const h8 hi0 = __builtin_bit_cast(h8, op[rpos]), lo0 = __builtin_bit_cast(h8, op[64 + rpos]);
                const int rpos1 = 16 * g + ((li + 2 * g + 8) & 15);
                const h8 hi1 = __builtin_bit_cast(h8, op[128 + rpos1]), lo1 = __builtin_bit_cast(h8, op[192 + rpos1]);
                const float inv = invs[buf * kInv + (i * T + t) * 16 + li];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const h8 w0 = __builtin_bit_cast(h8, wb[i][r][0]), w1 = __builtin_bit_cast(h8, wb[i][r][1]);
                    v4f m = __builtin_amdgcn_mfma_f32_16x16x32_f16(w0, hi0, v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                    m = __builtin_amdgcn_mfma_f32_16x16x32_f16(w1, hi1, m, 0, 0, 0);
                    m = __builtin_amdgcn_mfma_f32_16x16x32_f16(w0, lo0, m, 0, 0, 0);
                    m = __builtin_amdgcn_mfma_f32_16x16x32_f16(w1, lo1, m, 0, 0, 0);
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[r][t][e] = __fmaf_rn(m[e], inv, acc[r][t][e]);
                }
            }
            issue_w((c + 1) * C + i, i);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (c + 1 < chunks) stage_x(c + 1, buf ^ 1);
        __syncthreads();
    }
    if constexpr (Norm) {
        // Each token's squares: the 8 lanes of its values, then the staging
        // groups in order.
#pragma unroll
        for (int t = 0; t < T; ++t) {
            float v = ss[t];
            v += dev::xor_lane<1>(v);
            v += dev::xor_lane<2>(v);
            v += dev::xor_lane<4>(v);
            if (q8 == 0) sspart[gamma][t][tt] = v;
        }
        __syncthreads();
    }
    const uint32_t wrow = row0 + (uint32_t)wave * 16u * R;
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const uint32_t tok = tok0 + 16u * t + li;
        if (tok >= a.tokens) continue;
        float inv_rms = 1.0f;
        if constexpr (Norm) {
            float sum = sspart[0][t][li];
#pragma unroll
            for (int k = 1; k < kGroups; ++k) sum += sspart[k][t][li];
            inv_rms = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(sum, (float)a.cols), a.eps)));
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t rbase = wrow + 16u * r + 4u * g;
            float y[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) y[e] = Norm ? __fmul_rn(acc[r][t][e], inv_rms) : acc[r][t][e];
            if (a.pairs) {
#pragma unroll
                for (int e = 0; e < 4; e += 2)
                    if (rbase + e < a.rows)
                        a.out[(size_t)tok * (a.rows / 2) + (rbase + e) / 2] =
                            __fmul_rn(__fdiv_rn(y[e], __fadd_rn(1.0f, expf(-y[e]))), y[e + 1]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (rbase + e < a.rows) {
                        const size_t at = (size_t)tok * a.rows + rbase + e;
                        a.out[at] = a.residual ? a.residual[at] + y[e] : y[e];
                    }
            }
        }
    }
}

template <bool Norm, int R, int T, int W>
hipError_t launch_f16_rows(hipStream_t s, uint32_t tokens, const DenseArgs &a) {
    constexpr int C = 2;
    const dim3 grid((a.rows + 16 * R * W - 1) / (16 * R * W), (tokens + 16 * T - 1) / (16 * T));
    const size_t lds = (Norm ? (size_t)a.cols * 4 : 0) + 2 * ((size_t)C * T * 4 * 64 * 16 + (size_t)C * T * 16 * 4);
    void (*kernel)(const DenseArgs) = gemm_f16_rows_kernel<Norm, R, T, W>;
    if (lds > (48u << 10)) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kernel, grid, dim3(64 * W), lds, s, a);
    return hipGetLastError();
}

template <int TOK>
hipError_t launch_dense(hipStream_t s, dim3 grid, size_t lds, bool half, bool norm, const DenseArgs &a) {
    void (*kernel)(const DenseArgs) = half ? (norm ? gemv_dense_kernel<true, true, TOK> : gemv_dense_kernel<true, false, TOK>)
                                           : (norm ? gemv_dense_kernel<false, true, TOK> : gemv_dense_kernel<false, false, TOK>);
    if (lds > (64u << 10)) {
        // Beyond 64 KiB a launch's dynamic LDS has to be allowed per kernel.
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kernel, grid, dim3(256), lds, s, a);
    return hipGetLastError();
}

// From this many tokens the matrix-core form runs; its RMSNorm weights
// stay in LDS (the static tiles take about 5 KiB of the 160 KiB).
constexpr uint32_t kMmaMinTokens = 8;
constexpr uint32_t kMmaMaxNormCols = 36864;
constexpr size_t kMaxWorkgroupLds = 160u << 10;  // gfx950

// LDS of the f16 forms apart from RMSNorm weights: the rows form's two
// operand buffers and its per-group squares; the K-split form's
// activation tiles, partial tiles and squares (four wavefronts).
constexpr size_t rows_form_lds(int t, int w) {
    return 2 * ((size_t)2 * t * 4 * 64 * 16 + (size_t)2 * t * 16 * 4) + (size_t)(w / 2) * t * 16 * 4;
}
constexpr size_t ksplit_form_lds(int r) { return (size_t)4 * 16 * 17 * 16 + (size_t)4 * 16 * r * 17 * 4 + 4 * 16 * 4; }

hipError_t launch_mma(hipStream_t s, dim3 grid, size_t lds, bool half, bool norm, const DenseArgs &a) {
    void (*kernel)(const DenseArgs) = half ? (norm ? gemm_dense_kernel<true, true> : gemm_dense_kernel<true, false>)
                                           : (norm ? gemm_dense_kernel<false, true> : gemm_dense_kernel<false, false>);
    if (lds > (48u << 10)) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kernel, grid, dim3(256), lds, s, a);
    return hipGetLastError();
}

template <bool Norm, int R, int W, int D>
hipError_t launch_f16_mma(hipStream_t s, uint32_t tokens, size_t lds, const DenseArgs &a) {
    const dim3 grid((a.rows + 16 * R - 1) / (16 * R), (tokens + 15) / 16);
    void (*kernel)(const DenseArgs) = gemm_f16_kernel<Norm, R, W, D>;
    if (lds > (48u << 10)) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kernel, grid, dim3(64 * W), lds, s, a);
    return hipGetLastError();
}

// f16 bits of each value, round to nearest even (half_float.zig:12-16).
__global__ __launch_bounds__(256) void f32_to_f16_kernel(const float *in, uint64_t count, uint16_t *out) {
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < count; i += (uint64_t)gridDim.x * 256)
        out[i] = dev::f32_to_f16_bits(in[i]);
}

}  // namespace

bool gemv_dense_supported(int format, uint32_t cols) {
    return is_dense_format(format) && cols >= 1 && cols <= kDenseMaxCols;
}

hipError_t launch_gemv_dense(hipStream_t s, int cus, const GemvInput &in, const Matrix &w, uint32_t tokens,
                             float *out, const float *residual) {
    if (!gemv_dense_supported(w.format, w.cols) || tokens == 0) return hipErrorInvalidValue;
    if (in.mode != GemvInput::F32 && in.mode != GemvInput::RmsNorm) return hipErrorNotSupported;
    if ((in.pairs && ((w.rows & 1u) || residual)) || !in.x || !out || (in.mode == GemvInput::RmsNorm && !in.norm))
        return hipErrorInvalidValue;
    if (w.rows == 0) return hipSuccess;
    DenseArgs a{};
    a.w = w.data;
    a.rows = w.rows;
    a.cols = w.cols;
    a.tokens = tokens;
    a.x = in.x;
    a.norm = in.norm;
    a.eps = in.eps;
    a.out = out;
    a.residual = residual;
    a.pairs = in.pairs ? 1u : 0u;
    // Eight tokens and more: the matrix cores, the weights streamed once per
    // sixteen tokens (whole 16-byte loads of at least four K-steps per
    // wavefront, 16-byte aligned weights, activations and norm weights).
    const bool half = w.format == QWH_FORMAT_F16;
    const bool norm = in.mode == GemvInput::RmsNorm;
    const uint32_t step_cols = half ? 32u : 16u;
    const bool aligned = (((uintptr_t)w.data | (uintptr_t)in.x | (norm ? (uintptr_t)in.norm : 0u)) & 15u) == 0;
    if (tokens >= kMmaMinTokens && w.cols % step_cols == 0 && w.cols / step_cols >= 4 && aligned &&
        (!norm || w.cols <= kMmaMaxNormCols)) {
        const dim3 grid((w.rows + 15) / 16, (tokens + 15) / 16);
        if (grid.y > 65535) return hipErrorInvalidValue;
        const size_t lds = norm ? (size_t)w.cols * 4 : 0;
        if (half && w.cols % 64 == 0 && w.cols / 64 >= 4) {
            // f16 weights: the split-activation f16 forms, where their LDS
            // (with RMSNorm, the norm weights beside the operand buffers)
            // fits a workgroup's 160 KiB.
            const size_t norm_lds = norm ? (size_t)w.cols * 4 : 0;
            auto fits = [&](size_t bytes) { return norm_lds + bytes <= kMaxWorkgroupLds; };
            // More than 16 tokens: the rows form, T token tiles sharing each
            // weight load (measured best on the 1.7B shapes at 32 to 256
            // tokens and the lm_head at 64).
            if (tokens > 16) {
                if (w.rows < 8192) {
                    if (w.rows >= 4096 && fits(rows_form_lds(2, 8)))
                        return norm ? launch_f16_rows<true, 1, 2, 8>(s, tokens, a) : launch_f16_rows<false, 1, 2, 8>(s, tokens, a);
                    if (w.rows < 4096 && fits(rows_form_lds(2, 4)))
                        return norm ? launch_f16_rows<true, 1, 2, 4>(s, tokens, a) : launch_f16_rows<false, 1, 2, 4>(s, tokens, a);
                } else if (tokens >= 128 && fits(rows_form_lds(4, 8))) {
                    return norm ? launch_f16_rows<true, 2, 4, 8>(s, tokens, a) : launch_f16_rows<false, 2, 4, 8>(s, tokens, a);
                } else if (tokens < 128 && w.rows >= 65536 && fits(rows_form_lds(4, 8))) {
                    return norm ? launch_f16_rows<true, 1, 4, 8>(s, tokens, a) : launch_f16_rows<false, 1, 4, 8>(s, tokens, a);
                } else if (tokens < 128 && w.rows < 65536 && fits(rows_form_lds(2, 8))) {
                    return norm ? launch_f16_rows<true, 1, 2, 8>(s, tokens, a) : launch_f16_rows<false, 1, 2, 8>(s, tokens, a);
                }
            }
            // Up to 16 tokens (or rows-form LDS too large): K split over the
            // wavefronts, R row tiles per workgroup from the 16 x 16 tiles
            // per CU: up to 3, one workgroup per CU with that many (each
            // activation step then loaded once per CU: gate|up at 16 tokens
            // 18.7 -> 15.5 us with 3), else 4 (more rows per workgroup share
            // each activation load, several workgroups per CU).
            const uint64_t tiles = (uint64_t)grid.x * grid.y;
            const uint64_t cu = (uint64_t)(cus > 0 ? cus : 256);
            if (tiles > 3 * cu && fits(ksplit_form_lds(4)))
                return norm ? launch_f16_mma<true, 4, 4, 2>(s, tokens, lds, a) : launch_f16_mma<false, 4, 4, 2>(s, tokens, lds, a);
            if (tiles > 2 * cu && fits(ksplit_form_lds(3)))
                return norm ? launch_f16_mma<true, 3, 4, 2>(s, tokens, lds, a) : launch_f16_mma<false, 3, 4, 2>(s, tokens, lds, a);
            if (tiles > cu && fits(ksplit_form_lds(2)))
                return norm ? launch_f16_mma<true, 2, 4, 2>(s, tokens, lds, a) : launch_f16_mma<false, 2, 4, 2>(s, tokens, lds, a);
            if (fits(ksplit_form_lds(1)))
                return norm ? launch_f16_mma<true, 1, 4, 2>(s, tokens, lds, a) : launch_f16_mma<false, 1, 4, 2>(s, tokens, lds, a);
        }
        return launch_mma(s, grid, lds, half, norm, a);
    }
    // Tokens per workgroup (one pass over the weights per group): four from
    // three tokens on, two for two, each where its rows fit the LDS, else
    // the next smaller.
    int tok = 1;
    if (tokens >= 3 && w.cols <= dense_max_cols(4)) tok = 4;
    else if (tokens >= 2 && w.cols <= dense_max_cols(2)) tok = 2;
    const uint32_t groups = (tokens + tok - 1) / tok;
    if (groups > 65535) return hipErrorInvalidValue;
    // Workgroups per CU in all: eight for matrices of 128 MB and more (the
    // most weight bytes in flight) and for eight or more token groups (a
    // prompt's rows), four otherwise, where each workgroup's activation
    // prologue is worth spreading over more rows (measured on the 1.7B
    // decoder's matrices at batch 1 and 16, its prompt prefill and the 0.6B
    // lm_head shape).
    const uint32_t outputs = in.pairs ? w.rows / 2 : w.rows;
    const uint64_t wbytes = (uint64_t)w.rows * w.cols * dense_element_bytes(w.format);
    const uint32_t per_cu = wbytes >= (128ull << 20) || groups >= 8 ? 8u : 4u;
    const uint32_t target = (uint32_t)(cus > 0 ? cus : 256) * per_cu;
    uint32_t blocks = (target + groups - 1) / groups;
    const uint32_t most = (outputs + 3) / 4;
    if (blocks > most) blocks = most;
    if (blocks == 0) blocks = 1;
    const dim3 grid(blocks, groups);
    const size_t lds = (size_t)tok * ((size_t)w.cols + 4) * sizeof(float);
    if (tok == 4) return launch_dense<4>(s, grid, lds, half, norm, a);
    if (tok == 2) return launch_dense<2>(s, grid, lds, half, norm, a);
    return launch_dense<1>(s, grid, lds, half, norm, a);
}

hipError_t launch_f32_to_f16(hipStream_t s, const float *in, uint64_t count, uint16_t *out) {
    if (count == 0) return hipSuccess;
    uint64_t blocks = (count + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    f32_to_f16_kernel<<<(uint32_t)blocks, 256, 0, s>>>(in, count, out);
    return hipGetLastError();
}

}  // namespace qwh
