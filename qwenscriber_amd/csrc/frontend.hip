// The audio tower's convolution front end: model.zig:509-644 convolveAndPack
// and projectConvStep, with kernels.zig:302-427 conv3x3Stride2Gelu.
//
// The log-mel spectrogram is cut into chunks of 2 * n_window frames (the last
// one zero filled); each chunk goes through three 3x3, stride-2, padding-1
// convolutions with bias and GELU ([out][in][3][3] f16 weights, channel-major
// planes, as the checkpoint stores them); every valid time step of the third
// stage is flattened channel-major over the remaining frequency bins and
// projected by conv_out; the sinusoidal position of the step within its chunk
// (model.zig:751-763) is added.
//
// Convolution kernel: a workgroup computes 64 output channels over an 8 x 8
// tile of output positions of one image. The input channels go through LDS in
// stages of 8: the 17 x 17 input patch the tile reads (zero outside the
// plane, which is the padding) and the stage's weights as f32, laid out
// [channel][tap][output channel] so a thread reads its four output channels'
// weights with one 16-byte LDS load. A thread accumulates 4 output channels x
// 4 positions in f32 FMAs (the reference sums each input channel's nine taps
// before adding them to the output; the order here differs, within f32
// rounding), then adds the bias and applies GELU (the reference's erf fit).
#include <type_traits>

#include "common.h"
#include "device.h"

namespace qwh {
namespace {

constexpr int kOcTile = 64;    // output channels per workgroup
constexpr int kTile = 8;       // output rows and columns per workgroup
constexpr int kPatch = 2 * kTile + 1;
constexpr int kCi = 8;         // input channels per LDS stage

struct ConvArgs {
    float *out;                // [batch][out_ch][oh][ow]
    const float *in;           // [batch][in_ch][h][w]
    const uint16_t *weights;   // [out_ch][in_ch][9] f16 bits
    const float *bias;         // [out_ch]
    uint32_t out_ch, in_ch, h, w, oh, ow, tiles_w;
};

__global__ __launch_bounds__(256) void conv3x3s2_gelu_kernel(const ConvArgs a) {
    __shared__ float patch[kCi][kPatch * kPatch];
    __shared__ float4 wts[kCi][9][kOcTile / 4];
    const int t = threadIdx.x;
    const uint32_t oc0 = blockIdx.x * kOcTile;
    const uint32_t tile_r = blockIdx.y / a.tiles_w, tile_c = blockIdx.y % a.tiles_w;
    const uint32_t b = blockIdx.z;
    const int ocg = t >> 4;             // four output channels oc0 + 4 ocg ..
    const int pg = t & 15;              // four positions: tile row pg / 2, columns 4 (pg % 2) ..
    const int pr = pg >> 1, pc = (pg & 1) * 4;
    const int in_r0 = (int)(tile_r * kTile) * 2 - 1, in_c0 = (int)(tile_c * kTile) * 2 - 1;
    const float *in = a.in + (size_t)b * a.in_ch * a.h * a.w;
    float acc[4][4] = {};
    for (uint32_t ci0 = 0; ci0 < a.in_ch; ci0 += kCi) {
        __syncthreads();  // the previous stage's reads are done
        for (int i = t; i < kCi * kPatch * kPatch; i += 256) {
            const int c = i / (kPatch * kPatch), rem = i % (kPatch * kPatch);
            const int r = in_r0 + rem / kPatch, col = in_c0 + rem % kPatch;
            float v = 0.0f;
            if (ci0 + c < a.in_ch && r >= 0 && r < (int)a.h && col >= 0 && col < (int)a.w)
                v = in[((size_t)(ci0 + c) * a.h + r) * a.w + col];
            patch[c][rem] = v;
        }
        for (int i = t; i < kCi * 9 * kOcTile; i += 256) {
            const int oc = i % kOcTile, tap = (i / kOcTile) % 9, c = i / (kOcTile * 9);
            float v = 0.0f;
            if (ci0 + c < a.in_ch && oc0 + oc < a.out_ch)
                v = dev::f16_bits_to_f32(a.weights[((size_t)(oc0 + oc) * a.in_ch + ci0 + c) * 9 + tap]);
            reinterpret_cast<float *>(&wts[c][tap][0])[oc] = v;
        }
        __syncthreads();
        const int stage = a.in_ch - ci0 < (uint32_t)kCi ? (int)(a.in_ch - ci0) : kCi;
        for (int c = 0; c < stage; ++c) {
#pragma unroll
            for (int tap = 0; tap < 9; ++tap) {
                const int kh = tap / 3, kw = tap % 3;
                const float4 wv = wts[c][tap][ocg];
                const float *row = &patch[c][(2 * pr + kh) * kPatch + 2 * pc + kw];
                const float x[4] = {row[0], row[2], row[4], row[6]};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    acc[0][j] = fmaf(wv.x, x[j], acc[0][j]);
                    acc[1][j] = fmaf(wv.y, x[j], acc[1][j]);
                    acc[2][j] = fmaf(wv.z, x[j], acc[2][j]);
                    acc[3][j] = fmaf(wv.w, x[j], acc[3][j]);
                }
            }
        }
    }
    const uint32_t orow = tile_r * kTile + pr;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t oc = oc0 + 4 * ocg + k;
        if (oc >= a.out_ch || orow >= a.oh) continue;
        const float bias = a.bias[oc];
        float *dst = a.out + (((size_t)b * a.out_ch + oc) * a.oh + orow) * a.ow;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t ocol = tile_c * kTile + pc + j;
            if (ocol < a.ow) dst[ocol] = dev::gelu(bias + acc[k][j]);
        }
    }
}

// ---- Matrix-core form (input channels a multiple of 16) ----
//
// The convolution as an implicit GEMM on v_mfma_f32_32x32x16_bf16: rows are
// output channels, columns are output positions (row-major over the output
// plane), and the reduction runs over (tap, input channel) in stages of 16
// input channels, one 16-deep MFMA step per tap. Both operands are split into
// two bf16 terms: a weight (f16, 11 significant bits) is exactly hi + lo
// (hi = its bf16 rounding, lo = the exact remainder, at most 4 bits); an
// activation is hi + lo with hi its bf16 rounding and lo the bf16 rounding of
// the exact remainder (|x - hi - lo| <= 2^-17 |x|). The four products are
// accumulated in f32 by the MFMA, so each term is an exact product summed in
// f32: within 2^-17 of the f32 convolution per term, no overflow range of its
// own (bf16 has f32's exponent range).
//
// Workgroup: 128 output channels (four wavefronts of 32) x 64 positions (two
// 32-column MFMA tiles per wavefront, so each weight operand serves both).
// Per stage the 64 positions' input rows (at most 2 * ceil(63 / ow) + 3 of
// them, zero padding included) x 16 channels go into LDS as
// [row][col][channel] in both terms, double buffered, the next stage's values
// loaded into registers while this one multiplies. Weights come prepared
// [stage][tap][term][oc][16] (conv_mfma_prep_kernel) and each wavefront loads
// its 32 rows' 18 operands one stage ahead. (32-position workgroups measured
// 1.33 ms for the 30 s front end against 1.15 ms: every position tile reads
// the weights again.)
typedef __bf16 cbf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 cbf16x2 __attribute__((ext_vector_type(2)));
typedef float cf32x16 __attribute__((ext_vector_type(16)));

constexpr int kMfOc = 128;       // output channels per workgroup
constexpr int kMfPos = 64;       // output positions per workgroup (two 32-column MFMA tiles)
constexpr int kMfNt = kMfPos / 32;
constexpr int kMfIc = 16;        // input channels per stage
constexpr int kMfIcPad = 16;     // channel stride of a patch cell (bf16)
constexpr int kMfRounds = 4;     // patch items per thread at most (256 threads)
constexpr size_t kMfLdsMax = 80 * 1024;  // the patch buffers' LDS, two workgroups per CU

struct ConvMfmaArgs {
    float *out;                  // [batch][out_ch][oh * ow]
    const float *in;             // [batch][in_ch][h][w]
    const uint16_t *wprep;       // [in_ch / 16][9][2][oc_pad][16] bf16 bits
    const float *bias;
    uint32_t out_ch, oc_pad, in_ch, h, w, oh, ow, positions;
    uint32_t patch_rows, patch_cols;
};

// Prepared weights: f16 -> f32 (exact), hi = bf16(w), lo = bf16(w - hi)
// (exact), laid out for the A operand; rows past out_ch are zero.
__global__ void conv_mfma_prep_kernel(const uint16_t *weights, uint32_t out_ch, uint32_t oc_pad, uint32_t in_ch,
                                      uint16_t *wprep) {
    const uint64_t n = (uint64_t)oc_pad * in_ch * 9;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t icl = (uint32_t)(i % kMfIc);
        const uint32_t oc = (uint32_t)((i / kMfIc) % oc_pad);
        const uint32_t tap = (uint32_t)((i / ((uint64_t)kMfIc * oc_pad)) % 9);
        const uint32_t stage = (uint32_t)(i / ((uint64_t)kMfIc * oc_pad * 9));
        const uint32_t ic = stage * kMfIc + icl;
        const float v = oc < out_ch ? dev::f16_bits_to_f32(weights[((size_t)oc * in_ch + ic) * 9 + tap]) : 0.0f;
        const __bf16 hi = (__bf16)v;
        const __bf16 lo = (__bf16)(v - (float)hi);
        const size_t base = (((size_t)stage * 9 + tap) * 2) * oc_pad;
        wprep[(base + oc) * kMfIc + icl] = __builtin_bit_cast(uint16_t, hi);
        wprep[(base + oc_pad + oc) * kMfIc + icl] = __builtin_bit_cast(uint16_t, lo);
    }
}

__global__ __launch_bounds__(256) void conv3x3s2_gelu_mfma_kernel(const ConvMfmaArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint16_t patch_lds[];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const uint32_t oc0 = blockIdx.x * kMfOc + wave * 32;
    const uint32_t p0 = blockIdx.y * kMfPos;
    const uint32_t b = blockIdx.z;
    const uint32_t cells = a.patch_rows * a.patch_cols;
    const uint32_t term_elems = cells * kMfIcPad;          // one term of one buffer
    const uint32_t r_first = p0 / a.ow;
    const int in_r0 = 2 * (int)r_first - 1;                // input row of patch row 0
    const float *in = a.in + (size_t)b * a.in_ch * a.h * a.w;
    const uint32_t stages = a.in_ch / kMfIc;

    // B operand: this lane's position (column lane % 32) and channel half.
    uint32_t cell0[kMfNt];
#pragma unroll
    for (int j = 0; j < kMfNt; ++j) {
        uint32_t p = p0 + 32 * j + (lane & 31);
        if (p >= a.positions) p = a.positions - 1;              // (never stored)
        const uint32_t oh = p / a.ow, ow = p % a.ow;
        cell0[j] = (2 * (oh - r_first)) * a.patch_cols + 2 * ow;   // + kh * cols + kw
    }
    const uint32_t kq = (lane >> 5) * 8;
    // A operand: output channel oc0 + lane % 32, channels kq .. kq + 7.
    const uint16_t *wl = a.wprep + (size_t)(oc0 + (lane & 31)) * kMfIc + kq;
    const size_t wtap = (size_t)2 * a.oc_pad * kMfIc;      // elements per tap (both terms)
    const size_t wterm = (size_t)a.oc_pad * kMfIc;

    // Patch items: (channel half, row, col); a thread takes items
    // t, t + 256, ... (kMfRounds at most; the host checks 2 * cells fits).
    float stage_v[kMfRounds][8];
    auto load_patch = [&](uint32_t stage) {
#pragma unroll
        for (int k = 0; k < kMfRounds; ++k) {
            const uint32_t item = t + 256 * k;
            const uint32_t half = item / cells, cell = item % cells;
            const int r = in_r0 + (int)(cell / a.patch_cols);
            const int c = (int)(cell % a.patch_cols) - 1;
            const bool inside = half < 2 && r >= 0 && r < (int)a.h && c >= 0 && c < (int)a.w;
            const int rr = r < 0 ? 0 : (r >= (int)a.h ? (int)a.h - 1 : r);
            const int cc = c < 0 ? 0 : (c >= (int)a.w ? (int)a.w - 1 : c);
            const uint32_t ic = stage * kMfIc + (half < 2 ? half : 0) * 8;
            const float *src = in + ((size_t)ic * a.h + rr) * a.w + cc;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float v = src[(size_t)j * a.h * a.w];   // (unconditional: clamped inside the plane)
                stage_v[k][j] = inside ? v : 0.0f;
            }
        }
    };
    auto store_patch = [&](int buf) {
        uint16_t *hi_base = patch_lds + (size_t)buf * 2 * term_elems;
        uint16_t *lo_base = hi_base + term_elems;
#pragma unroll
        for (int k = 0; k < kMfRounds; ++k) {
            const uint32_t item = t + 256 * k;
            if (item >= 2 * cells) break;
            const uint32_t half = item / cells, cell = item % cells;
            uint32_t hw[4], lw[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float x0 = stage_v[k][2 * j], x1 = stage_v[k][2 * j + 1];
                const cbf16x2 h2 = {(__bf16)x0, (__bf16)x1};
                const cbf16x2 l2 = {(__bf16)(x0 - (float)h2[0]), (__bf16)(x1 - (float)h2[1])};
                hw[j] = __builtin_bit_cast(uint32_t, h2);
                lw[j] = __builtin_bit_cast(uint32_t, l2);
            }
            const size_t at = (size_t)cell * kMfIcPad + half * 8;
            *reinterpret_cast<uint4 *>(hi_base + at) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
            *reinterpret_cast<uint4 *>(lo_base + at) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
        }
    };
    cbf16x8 wa[2][9][2];  // [stage buffer][tap][term]
    auto load_weights = [&](uint32_t stage, int buf) {
        const uint16_t *src = wl + (size_t)stage * 9 * wtap;
#pragma unroll
        for (int tap = 0; tap < 9; ++tap)
#pragma unroll
            for (int term = 0; term < 2; ++term)
                wa[buf][tap][term] = *reinterpret_cast<const cbf16x8 *>(src + tap * wtap + term * wterm);
    };

    cf32x16 acc[kMfNt] = {}, acc2[kMfNt] = {};
    // One stage: the next stage's values and weights are loaded (the last
    // stage reloads its own: the loads stay unconditional), this stage is
    // multiplied out of LDS buffer BUF, and the next stage's values go into
    // the other buffer; every wavefront read that buffer in the previous
    // stage, before the barrier that ended it.
    auto stage_step = [&](uint32_t s, auto buf_tag) {
        constexpr int BUF = decltype(buf_tag)::value;
        const uint32_t nxt = s + 1 < stages ? s + 1 : s;
        load_patch(nxt);
        load_weights(nxt, BUF ^ 1);
        __builtin_amdgcn_sched_barrier(0);
        const uint16_t *hb = patch_lds + (size_t)BUF * 2 * term_elems;
        const uint16_t *lb = hb + term_elems;
#pragma unroll
        for (int tap = 0; tap < 9; ++tap) {
#pragma unroll
            for (int j = 0; j < kMfNt; ++j) {
                const uint32_t cell = cell0[j] + (tap / 3) * a.patch_cols + (tap % 3);
                const cbf16x8 bh = *reinterpret_cast<const cbf16x8 *>(hb + (size_t)cell * kMfIcPad + kq);
                const cbf16x8 bl = *reinterpret_cast<const cbf16x8 *>(lb + (size_t)cell * kMfIcPad + kq);
                // (Two accumulators, so consecutive products do not wait on
                // each other's results.)
                acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wa[BUF][tap][0], bh, acc[j], 0, 0, 0);
                acc2[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wa[BUF][tap][0], bl, acc2[j], 0, 0, 0);
                acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wa[BUF][tap][1], bh, acc[j], 0, 0, 0);
                acc2[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wa[BUF][tap][1], bl, acc2[j], 0, 0, 0);
            }
        }
        store_patch(BUF ^ 1);
        __syncthreads();
    };
    load_patch(0);
    load_weights(0, 0);
    store_patch(0);
    __syncthreads();
    uint32_t s = 0;
    for (; s + 1 < stages; s += 2) {
        stage_step(s, std::integral_constant<int, 0>{});
        stage_step(s + 1, std::integral_constant<int, 1>{});
    }
    if (s < stages) stage_step(s, std::integral_constant<int, 0>{});
    // Value r of a lane: output channel row 8 (r / 4) + 4 (lane / 32) + r % 4
    // of the wavefront's 32, position column lane % 32.
#pragma unroll
    for (int j = 0; j < kMfNt; ++j) {
        const uint32_t pos = p0 + 32 * j + (lane & 31);
        if (pos >= a.positions) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t oc = oc0 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
            if (oc < a.out_ch)
                a.out[((size_t)b * a.out_ch + oc) * a.positions + pos] =
                    dev::gelu(a.bias[oc] + (acc[j][r] + acc2[j][r]));
        }
    }
}

// One input channel (conv1 of the tower, on the log-mel): each thread takes
// one output position of one image and a range of output channels; its nine
// input samples are read once, each output is bias + the taps in the
// reference's order (rows, then columns; taps outside the plane skipped),
// then GELU. Stores are coalesced over positions.
constexpr uint32_t kC1Oc = 64;   // output channels per workgroup column
__global__ __launch_bounds__(256) void conv1_gelu_kernel(const ConvArgs a) {
    __shared__ float wts[kC1Oc][9];
    __shared__ float bs[kC1Oc];
    const uint32_t t = threadIdx.x;
    const uint32_t oc0 = blockIdx.y * kC1Oc;
    const uint32_t b = blockIdx.z;
    const uint32_t positions = a.oh * a.ow;
    const uint32_t p = blockIdx.x * 256 + t;
    for (uint32_t i = t; i < kC1Oc * 9; i += 256) {
        const uint32_t oc = oc0 + i / 9;
        wts[i / 9][i % 9] = oc < a.out_ch ? dev::f16_bits_to_f32(a.weights[(size_t)oc * 9 + i % 9]) : 0.0f;
    }
    if (t < kC1Oc) bs[t] = oc0 + t < a.out_ch ? a.bias[oc0 + t] : 0.0f;
    __syncthreads();
    if (p >= positions) return;
    const uint32_t orow = p / a.ow, ocol = p % a.ow;
    const float *in = a.in + (size_t)b * a.h * a.w;
    float x[9];
    bool ok[9];
#pragma unroll
    for (int tap = 0; tap < 9; ++tap) {
        const int r = (int)orow * 2 + tap / 3 - 1, c = (int)ocol * 2 + tap % 3 - 1;
        ok[tap] = r >= 0 && r < (int)a.h && c >= 0 && c < (int)a.w;
        x[tap] = ok[tap] ? in[(size_t)r * a.w + c] : 0.0f;
    }
    const uint32_t end = a.out_ch - oc0 < kC1Oc ? a.out_ch - oc0 : kC1Oc;
    float *out = a.out + ((size_t)b * a.out_ch + oc0) * positions + p;
    for (uint32_t k = 0; k < end; ++k) {
        float acc = 0.0f;
#pragma unroll
        for (int tap = 0; tap < 9; ++tap)
            if (ok[tap]) acc = fmaf(wts[k][tap], x[tap], acc);
        out[(size_t)k * positions] = dev::gelu(bs[k] + acc);
    }
}

// Chunks [first, first + count) of the log-mel [bins][frames] into
// [count][bins][chunk_frames], frames past the clip zero (model.zig:557-563).
__global__ void gather_chunks_kernel(const float *mel, uint32_t bins, uint32_t frames, uint32_t chunk_frames,
                                     uint32_t first, uint32_t count, float *out) {
    const uint64_t n = (uint64_t)count * bins * chunk_frames;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t t = (uint32_t)(i % chunk_frames);
        const uint32_t bin = (uint32_t)((i / chunk_frames) % bins);
        const uint32_t c = (uint32_t)(i / ((uint64_t)chunk_frames * bins));
        const uint64_t frame = (uint64_t)(first + c) * chunk_frames + t;
        out[i] = frame < frames ? mel[(uint64_t)bin * frames + frame] : 0.0f;
    }
}

// projectConvStep's flatten (model.zig:615-631). Every chunk but the clip's
// last is whole, so row r of a run of chunks is step r % steps_per_chunk of
// chunk r / steps_per_chunk; its features are channel-major over the
// frequency bins: flat[r][c * bins + f] = conv3[chunk][c][f][step].
__global__ void pack_steps_kernel(const float *conv3, uint32_t channels, uint32_t bins, uint32_t steps_per_chunk,
                                  uint32_t rows, float *flat) {
    const uint32_t features = channels * bins;
    const uint64_t n = (uint64_t)rows * features;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t r = (uint32_t)(i / features), k = (uint32_t)(i % features);
        const uint32_t c = k / bins, f = k % bins;
        const uint32_t chunk = r / steps_per_chunk, step = r % steps_per_chunk;
        flat[i] = conv3[(((uint64_t)chunk * channels + c) * bins + f) * steps_per_chunk + step];
    }
}

// addSinusoidalPosition (model.zig:751-763) from a table of f32 values the
// host computed in f64: encoder row first + r is step (first + r) %
// steps_per_chunk of its chunk.
__global__ void add_positions_kernel(float *rows, const float *table, uint32_t first, uint32_t count, uint32_t width,
                                     uint32_t steps_per_chunk) {
    const uint64_t n = (uint64_t)count * width;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t r = (uint32_t)(i / width), k = (uint32_t)(i % width);
        rows[i] += table[(uint64_t)((first + r) % steps_per_chunk) * width + k];
    }
}

unsigned blocks_for(uint64_t n) {
    const uint64_t b = (n + 255) / 256;
    return (unsigned)(b < 65535 ? (b ? b : 1) : 65535);
}

}  // namespace

hipError_t launch_conv3x3s2_gelu(hipStream_t s, float *out, const float *in, const uint16_t *weights, const float *bias,
                                 uint32_t batch, uint32_t out_ch, uint32_t in_ch, uint32_t h, uint32_t w) {
    ConvArgs a{};
    a.out = out, a.in = in, a.weights = weights, a.bias = bias;
    a.out_ch = out_ch, a.in_ch = in_ch, a.h = h, a.w = w;
    a.oh = (h - 1) / 2 + 1, a.ow = (w - 1) / 2 + 1;
    a.tiles_w = (a.ow + kTile - 1) / kTile;
    const uint32_t tiles_h = (a.oh + kTile - 1) / kTile;
    if (in_ch == 1) {
        const dim3 grid1((a.oh * a.ow + 255) / 256, (out_ch + kC1Oc - 1) / kC1Oc, batch);
        conv1_gelu_kernel<<<grid1, 256, 0, s>>>(a);
        return hipGetLastError();
    }
    const dim3 grid((out_ch + kOcTile - 1) / kOcTile, tiles_h * a.tiles_w, batch);
    conv3x3s2_gelu_kernel<<<grid, 256, 0, s>>>(a);
    return hipGetLastError();
}

namespace {

// Patch rows for kMfPos positions starting anywhere in a row of `ow`.
uint32_t mfma_patch_rows(uint32_t ow) { return 2 * ((kMfPos - 1 + ow - 1) / ow) + 3; }

}  // namespace

size_t conv_mfma_prep_bytes(uint32_t out_ch, uint32_t in_ch) {
    const uint32_t oc_pad = (out_ch + kMfOc - 1) / kMfOc * kMfOc;
    return (size_t)oc_pad * in_ch * 9 * 2 * sizeof(uint16_t);
}

bool conv_mfma_supported(uint32_t in_ch, uint32_t h, uint32_t w) {
    if (in_ch == 0 || in_ch % kMfIc || h == 0 || w == 0) return false;
    const uint32_t ow = (w - 1) / 2 + 1;
    const uint64_t cells = (uint64_t)mfma_patch_rows(ow) * (w + 2);
    // Two channel halves per cell in kMfRounds rounds of 256 threads; two
    // buffers of two terms in LDS.
    return 2 * cells <= 256u * kMfRounds && cells * kMfIcPad * 2 * 2 * sizeof(uint16_t) <= kMfLdsMax;
}

hipError_t launch_conv_mfma_prep(hipStream_t s, const uint16_t *weights, uint32_t out_ch, uint32_t in_ch, void *wprep) {
    const uint32_t oc_pad = (out_ch + kMfOc - 1) / kMfOc * kMfOc;
    conv_mfma_prep_kernel<<<blocks_for((uint64_t)oc_pad * in_ch * 9), 256, 0, s>>>(weights, out_ch, oc_pad, in_ch,
                                                                                   static_cast<uint16_t *>(wprep));
    return hipGetLastError();
}

hipError_t launch_conv3x3s2_gelu_mfma(hipStream_t s, float *out, const float *in, const void *wprep, const float *bias,
                                     uint32_t batch, uint32_t out_ch, uint32_t in_ch, uint32_t h, uint32_t w) {
    if (!conv_mfma_supported(in_ch, h, w) || batch == 0 || batch > 65535) return hipErrorInvalidValue;
    ConvMfmaArgs a{};
    a.out = out, a.in = in, a.wprep = static_cast<const uint16_t *>(wprep), a.bias = bias;
    a.out_ch = out_ch, a.oc_pad = (out_ch + kMfOc - 1) / kMfOc * kMfOc, a.in_ch = in_ch, a.h = h, a.w = w;
    a.oh = (h - 1) / 2 + 1, a.ow = (w - 1) / 2 + 1;
    a.positions = a.oh * a.ow;
    a.patch_rows = mfma_patch_rows(a.ow);
    a.patch_cols = w + 2;
    const size_t lds = (size_t)a.patch_rows * a.patch_cols * kMfIcPad * 2 * 2 * sizeof(uint16_t);
    // (Above the default 64 KB of dynamic LDS: raised once, to the most any
    // supported shape asks for.)
    static const hipError_t raised = hipFuncSetAttribute(reinterpret_cast<const void *>(&conv3x3s2_gelu_mfma_kernel),
                                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMfLdsMax);
    if (raised != hipSuccess) return raised;
    const dim3 grid(a.oc_pad / kMfOc, (a.positions + kMfPos - 1) / kMfPos, batch);
    conv3x3s2_gelu_mfma_kernel<<<grid, 256, lds, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_gather_chunks(hipStream_t s, const float *mel, uint32_t bins, uint32_t frames, uint32_t chunk_frames,
                                uint32_t first, uint32_t count, float *out) {
    gather_chunks_kernel<<<blocks_for((uint64_t)count * bins * chunk_frames), 256, 0, s>>>(mel, bins, frames, chunk_frames,
                                                                                          first, count, out);
    return hipGetLastError();
}

hipError_t launch_pack_steps(hipStream_t s, const float *conv3, uint32_t channels, uint32_t bins, uint32_t steps_per_chunk,
                             uint32_t rows, float *flat) {
    pack_steps_kernel<<<blocks_for((uint64_t)rows * channels * bins), 256, 0, s>>>(conv3, channels, bins,
                                                                                  steps_per_chunk, rows, flat);
    return hipGetLastError();
}

hipError_t launch_add_positions(hipStream_t s, float *rows, const float *table, uint32_t first, uint32_t count,
                                uint32_t width, uint32_t steps_per_chunk) {
    add_positions_kernel<<<blocks_for((uint64_t)count * width), 256, 0, s>>>(rows, table, first, count, width,
                                                                            steps_per_chunk);
    return hipGetLastError();
}

}  // namespace qwh
