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
    const dim3 grid((out_ch + kOcTile - 1) / kOcTile, tiles_h * a.tiles_w, batch);
    conv3x3s2_gelu_kernel<<<grid, 256, 0, s>>>(a);
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
