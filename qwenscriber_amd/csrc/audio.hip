// Audio tower glue and windowed encoder attention for gfx950.
//
// The audio tower (model.zig:646-705 runAudioTower) runs its projections
// through the same quantized linear as the decoder; what it adds around them
// is restated here:
//   - LayerNorm with bias (math.zig:99-116, kernels.zig:242-271);
//   - bias epilogues: addBias (kernels.zig:210-218), bias then exact GELU
//     (math.zig:46-66, model.zig:717-719 / :866-868), bias then residual add
//     (model.zig:824-848 + :669 addInPlace);
//   - non-causal attention inside fixed windows of steps
//     (kernels.zig:429-484 audioAttentionWindow, model.zig:792-822).
//
// Every kernel is HBM/latency bound at the audio tower's sizes (at 30 s of
// audio 390 steps x 896..1024 channels, 1.4-1.6 MB per activation plane), so
// the layouts follow the reference's row-major [step][channel] buffers and the
// kernels only make sure every load is coalesced.

#include "common.h"
#include "device.h"

namespace qwh {

namespace {

constexpr int kNormThreads = 256;

// Sum over a 256-thread workgroup; every thread gets the total.
__device__ __forceinline__ float block_sum_256(float v, float *lds) {
    v = dev::wave_sum(v);
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) lds[wave] = v;
    __syncthreads();
    return (lds[0] + lds[1]) + (lds[2] + lds[3]);
}

// LayerNorm of one row per workgroup: mean, centred variance,
// 1 / sqrt(variance + eps), then (x - mean) * inverse_std * weight + bias.
// `out` may alias `x` (each thread rewrites only the elements it read last).
__global__ __launch_bounds__(kNormThreads) void layer_norm_kernel(const float *x, float *out, const float *weight,
                                                                  const float *bias, uint32_t width, float eps) {
    __shared__ float lds[4];
    const float *row = x + (size_t)blockIdx.x * width;
    float *dst = out + (size_t)blockIdx.x * width;
    float sum = 0.0f;
    for (uint32_t i = threadIdx.x; i < width; i += kNormThreads) sum += row[i];
    const float mean = block_sum_256(sum, lds) / (float)width;
    float squares = 0.0f;
    for (uint32_t i = threadIdx.x; i < width; i += kNormThreads) {
        const float centered = row[i] - mean;
        squares += centered * centered;
    }
    const float variance = block_sum_256(squares, lds) / (float)width;
    const float inverse_std = 1.0f / sqrtf(variance + eps);
    for (uint32_t i = threadIdx.x; i < width; i += kNormThreads)
        dst[i] = (row[i] - mean) * inverse_std * weight[i] + bias[i];
}

// The reference's erf (math.zig:46-60): the Numerical Recipes Chebyshev fit
// of erfc (`erfcc`), evaluated in f32 by Horner's rule.
__device__ __forceinline__ float erf_fit(float x) {
    const float magnitude = fabsf(x);
    const float t = 1.0f / (1.0f + 0.5f * magnitude);
    float poly = -0.82215223f + t * 0.17087277f;
    poly = 1.48851587f + t * poly;
    poly = -1.13520398f + t * poly;
    poly = 0.27886807f + t * poly;
    poly = -0.18628806f + t * poly;
    poly = 0.09678418f + t * poly;
    poly = 0.37409196f + t * poly;
    poly = 1.00002368f + t * poly;
    const float tau = t * expf(-magnitude * magnitude - 1.26551223f + t * poly);
    return copysignf(1.0f - tau, x);
}

__device__ __forceinline__ float gelu(float x) { return 0.5f * x * (1.0f + erf_fit(x * 0.70710678f)); }

// x[t][r] + bias[r], then per mode: stored (addBias), GELU of it stored, or
// added onto `residual` (x left as it was). `bias` may be null (no bias).
template <int Mode>
__global__ __launch_bounds__(256) void bias_epilogue_kernel(float *x, const float *bias, float *residual,
                                                            uint32_t rows, uint64_t total) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        float v = x[i];
        if (bias) v += bias[i % rows];
        if constexpr (Mode == kBiasAdd) x[i] = v;
        if constexpr (Mode == kBiasGelu) x[i] = gelu(v);
        if constexpr (Mode == kBiasResidual) residual[i] = residual[i] + v;
    }
}

// Windowed attention. Workgroup (query tile, window, head): 64 queries of
// one window and head, G = HD / 32 lanes per query, each lane owning 32 of
// the head's dimensions. Keys and values of the window pass through LDS in
// chunks of 64 rows; each query keeps an online softmax (running maximum,
// running sum, 32 accumulators per lane) and divides once at the end, which
// equals softmax-then-weighted-sum up to f32 rounding.
constexpr int kQueriesPerTile = 64;
constexpr int kKeysPerChunk = 64;

template <int HD>
__global__ __launch_bounds__(kQueriesPerTile *(HD / 32)) void audio_attention_kernel(AudioAttentionArgs a) {
    constexpr int G = HD / 32;
    constexpr int kThreads = kQueriesPerTile * G;
    constexpr int kRow = HD + 4;  // LDS row pitch in floats (16-byte aligned, staggered banks)
    __shared__ float4 lds_k[kKeysPerChunk * kRow / 4];
    __shared__ float4 lds_v[kKeysPerChunk * kRow / 4];
    const float *ks = reinterpret_cast<const float *>(lds_k);
    const float *vs = reinterpret_cast<const float *>(lds_v);

    const uint32_t start = a.first + blockIdx.y * a.window_steps;
    if (start >= a.end) return;
    const uint32_t length = min(a.window_steps, a.end - start);
    const uint32_t q0 = blockIdx.x * kQueriesPerTile;
    if (q0 >= length) return;
    const uint32_t head = blockIdx.z;
    const uint32_t column = head * HD;

    const int lane = threadIdx.x;
    const uint32_t query = q0 + lane / G;
    const int part = lane % G;
    const bool valid = query < length;
    const uint32_t query_row = start + (valid ? query : length - 1);

    float qv[32];
    {
        const float4 *src = reinterpret_cast<const float4 *>(a.q + (size_t)query_row * a.q_stride + column + part * 32);
        const float4 *qb = a.q_bias ? reinterpret_cast<const float4 *>(a.q_bias + column + part * 32) : nullptr;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float4 v = src[i];
            if (qb) {
                const float4 b = qb[i];
                v.x += b.x, v.y += b.y, v.z += b.z, v.w += b.w;
            }
            qv[4 * i] = v.x, qv[4 * i + 1] = v.y, qv[4 * i + 2] = v.z, qv[4 * i + 3] = v.w;
        }
    }
    float acc[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) acc[i] = 0.0f;
    float running_max = -INFINITY, running_sum = 0.0f;

    for (uint32_t k0 = 0; k0 < length; k0 += kKeysPerChunk) {
        const uint32_t count = min((uint32_t)kKeysPerChunk, length - k0);
        __syncthreads();
        for (int idx = threadIdx.x; idx < kKeysPerChunk * (HD / 4); idx += kThreads) {
            const int r = idx / (HD / 4), c = (idx % (HD / 4)) * 4;
            const uint32_t row = start + k0 + min((uint32_t)r, count - 1);
            float4 kv = *reinterpret_cast<const float4 *>(a.k + (size_t)row * a.k_stride + column + c);
            float4 vv = *reinterpret_cast<const float4 *>(a.v + (size_t)row * a.v_stride + column + c);
            if (a.k_bias) {
                const float4 b = *reinterpret_cast<const float4 *>(a.k_bias + column + c);
                kv.x += b.x, kv.y += b.y, kv.z += b.z, kv.w += b.w;
            }
            if (a.v_bias) {
                const float4 b = *reinterpret_cast<const float4 *>(a.v_bias + column + c);
                vv.x += b.x, vv.y += b.y, vv.z += b.z, vv.w += b.w;
            }
            lds_k[(r * kRow + c) / 4] = kv;
            lds_v[(r * kRow + c) / 4] = vv;
        }
        __syncthreads();
        for (uint32_t j = 0; j < count; ++j) {
            const float4 *krow = reinterpret_cast<const float4 *>(ks + j * kRow + part * 32);
            float dot = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float4 kk = krow[i];
                dot += qv[4 * i] * kk.x + qv[4 * i + 1] * kk.y + qv[4 * i + 2] * kk.z + qv[4 * i + 3] * kk.w;
            }
            const float score = dev::group_sum<G>(dot) * a.scaling;
            if (score > running_max) {
                const float correction = expf(running_max - score);
                running_sum *= correction;
#pragma unroll
                for (int i = 0; i < 32; ++i) acc[i] *= correction;
                running_max = score;
            }
            const float p = expf(score - running_max);
            running_sum += p;
            const float4 *vrow = reinterpret_cast<const float4 *>(vs + j * kRow + part * 32);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float4 vv = vrow[i];
                acc[4 * i] += p * vv.x, acc[4 * i + 1] += p * vv.y;
                acc[4 * i + 2] += p * vv.z, acc[4 * i + 3] += p * vv.w;
            }
        }
    }
    if (!valid) return;
    const float inverse = 1.0f / running_sum;
    float4 *dst = reinterpret_cast<float4 *>(a.out + (size_t)(start + query) * a.out_stride + column + part * 32);
#pragma unroll
    for (int i = 0; i < 8; ++i)
        dst[i] = make_float4(acc[4 * i] * inverse, acc[4 * i + 1] * inverse, acc[4 * i + 2] * inverse,
                             acc[4 * i + 3] * inverse);
}

}  // namespace

hipError_t launch_layer_norm(hipStream_t s, const float *x, float *out, const float *weight, const float *bias,
                             uint32_t width, uint32_t tokens, float eps) {
    if (tokens == 0) return hipSuccess;
    layer_norm_kernel<<<tokens, kNormThreads, 0, s>>>(x, out, weight, bias, width, eps);
    return hipGetLastError();
}

hipError_t launch_bias_epilogue(hipStream_t s, int mode, float *x, const float *bias, float *residual, uint32_t rows,
                                uint32_t tokens) {
    const uint64_t total = (uint64_t)rows * tokens;
    if (total == 0) return hipSuccess;
    const uint32_t blocks = (uint32_t)std::min<uint64_t>((total + 255) / 256, 4096);
    switch (mode) {
    case kBiasAdd: bias_epilogue_kernel<kBiasAdd><<<blocks, 256, 0, s>>>(x, bias, residual, rows, total); break;
    case kBiasGelu: bias_epilogue_kernel<kBiasGelu><<<blocks, 256, 0, s>>>(x, bias, residual, rows, total); break;
    case kBiasResidual:
        bias_epilogue_kernel<kBiasResidual><<<blocks, 256, 0, s>>>(x, bias, residual, rows, total);
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

bool audio_attention_supported(uint32_t head_dim) { return head_dim == 32 || head_dim == 64 || head_dim == 128; }

hipError_t launch_audio_attention(hipStream_t s, const AudioAttentionArgs &a) {
    if (a.end <= a.first || a.window_steps == 0 || a.heads == 0) return hipSuccess;
    const uint32_t span = a.end - a.first;
    const uint32_t windows = (span + a.window_steps - 1) / a.window_steps;
    const uint32_t longest = std::min(a.window_steps, span);
    const dim3 grid((longest + kQueriesPerTile - 1) / kQueriesPerTile, windows, a.heads);
    switch (a.head_dim) {
    case 32: audio_attention_kernel<32><<<grid, kQueriesPerTile * 1, 0, s>>>(a); break;
    case 64: audio_attention_kernel<64><<<grid, kQueriesPerTile * 2, 0, s>>>(a); break;
    case 128: audio_attention_kernel<128><<<grid, kQueriesPerTile * 4, 0, s>>>(a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace qwh
