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

// LayerNorm of one row per workgroup: mean, centred variance,
// 1 / sqrt(variance + eps), then (x - mean) * inverse_std * weight + bias.
// `out` may alias `x` (each thread rewrites only the elements it read last).
__global__ __launch_bounds__(kNormThreads) void layer_norm_kernel(const float *x, float *out, const float *weight,
                                                                  const float *bias, uint32_t width, float eps) {
    __shared__ float lds[4];
    const float *row = x + (size_t)blockIdx.x * width;
    float *dst = out + (size_t)blockIdx.x * width;
    float mean, inverse_std;
    dev::layer_norm_stats(row, width, eps, lds, mean, inverse_std);
    for (uint32_t i = threadIdx.x; i < width; i += kNormThreads)
        dst[i] = (row[i] - mean) * inverse_std * weight[i] + bias[i];
}

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
        if constexpr (Mode == kBiasGelu) x[i] = dev::gelu(v);
        if constexpr (Mode == kBiasResidual) residual[i] = residual[i] + v;
    }
}

// Windowed attention. One workgroup per (query tile, window, head) of
// kWaves wavefronts: G = HD / 16 lanes per query, each lane owning 16 of the
// head's dimensions, so a tile is 64 / G queries, and every wavefront holds
// the whole tile. Keys and values of the window pass through LDS in chunks of
// 64 rows; the wavefronts split each chunk's keys four ways (lanes of one
// query read different slices, the tile's queries the same ones:
// broadcasts). Each wavefront keeps an online softmax per query (running
// maximum, running sum, 16 accumulators per lane), two keys per step so
// their dot products, reductions and exponentials overlap; at the end the
// four partial states are merged through LDS and divided once:
// softmax-then-weighted-sum up to f32 rounding.
constexpr int kDimsPerLane = 16;
constexpr int kKeysPerChunk = 64;
constexpr int kWaves = 4;

template <int HD>
struct AudioTile {
    static constexpr int G = HD / kDimsPerLane;
    static constexpr int queries = 64 / G;
};

__device__ __forceinline__ float slice_dot(const float (&qv)[kDimsPerLane], const float *krow) {
    const float4 *k4 = reinterpret_cast<const float4 *>(krow);
    float even = 0.0f, odd = 0.0f;
#pragma unroll
    for (int i = 0; i < kDimsPerLane / 4; i += 2) {
        const float4 a = k4[i], b = k4[i + 1];
        even += qv[4 * i] * a.x + qv[4 * i + 1] * a.y + qv[4 * i + 2] * a.z + qv[4 * i + 3] * a.w;
        odd += qv[4 * i + 4] * b.x + qv[4 * i + 5] * b.y + qv[4 * i + 6] * b.z + qv[4 * i + 7] * b.w;
    }
    return even + odd;
}

struct SoftmaxState {
    float max = -INFINITY, sum = 0.0f;
    float acc[kDimsPerLane];
};

// Folds scores s0 (and s1 when `two`) with value rows v0 / v1 into the state.
template <bool two>
__device__ __forceinline__ void softmax_fold(SoftmaxState &st, float s0, float s1, const float *v0, const float *v1) {
    const float top = two ? fmaxf(s0, s1) : s0;
    if (top > st.max) {
        const float correction = expf(st.max - top);
        st.sum *= correction;
#pragma unroll
        for (int i = 0; i < kDimsPerLane; ++i) st.acc[i] *= correction;
        st.max = top;
    }
    const float p0 = expf(s0 - st.max);
    st.sum += p0;
    const float4 *x4 = reinterpret_cast<const float4 *>(v0);
    if constexpr (two) {
        const float p1 = expf(s1 - st.max);
        st.sum += p1;
        const float4 *y4 = reinterpret_cast<const float4 *>(v1);
#pragma unroll
        for (int i = 0; i < kDimsPerLane / 4; ++i) {
            const float4 x = x4[i], y = y4[i];
            st.acc[4 * i] += p0 * x.x + p1 * y.x;
            st.acc[4 * i + 1] += p0 * x.y + p1 * y.y;
            st.acc[4 * i + 2] += p0 * x.z + p1 * y.z;
            st.acc[4 * i + 3] += p0 * x.w + p1 * y.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < kDimsPerLane / 4; ++i) {
            const float4 x = x4[i];
            st.acc[4 * i] += p0 * x.x, st.acc[4 * i + 1] += p0 * x.y;
            st.acc[4 * i + 2] += p0 * x.z, st.acc[4 * i + 3] += p0 * x.w;
        }
    }
}

template <int HD>
__global__ __launch_bounds__(64 * kWaves) void audio_attention_kernel(AudioAttentionArgs a) {
    constexpr int G = AudioTile<HD>::G;
    constexpr int QT = AudioTile<HD>::queries;
    constexpr int kRow = HD + 4;  // LDS row pitch in floats (16-byte aligned, staggered banks)
    constexpr int kState = 4 + kDimsPerLane;  // max, sum, two pad, accumulators
    // Keys, then values, of one chunk; after the last chunk the same space
    // holds the wavefronts' merge records.
    constexpr int kChunkFloats = kKeysPerChunk * kRow;
    constexpr int kRecordFloats = kWaves * 64 * kState;
    constexpr int kLdsFloats = 2 * kChunkFloats > kRecordFloats ? 2 * kChunkFloats : kRecordFloats;
    __shared__ float4 lds[kLdsFloats / 4];
    float4 *lds_k = lds;
    float4 *lds_v = lds + kChunkFloats / 4;
    const float *ks = reinterpret_cast<const float *>(lds_k);
    const float *vs = reinterpret_cast<const float *>(lds_v);

    const uint32_t start = a.first + blockIdx.y * a.window_steps;
    if (start >= a.end) return;
    const uint32_t length = min(a.window_steps, a.end - start);
    const uint32_t q0 = blockIdx.x * QT;
    if (q0 >= length) return;
    const uint32_t column = blockIdx.z * HD;

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const uint32_t query = q0 + lane / G;
    const int slice = (lane % G) * kDimsPerLane;
    const bool valid = query < length;
    const uint32_t query_row = start + (valid ? query : length - 1);

    float qv[kDimsPerLane];
    {
        const float4 *src = reinterpret_cast<const float4 *>(a.q + (size_t)query_row * a.q_stride + column + slice);
        const float4 *qb = a.q_bias ? reinterpret_cast<const float4 *>(a.q_bias + column + slice) : nullptr;
#pragma unroll
        for (int i = 0; i < kDimsPerLane / 4; ++i) {
            float4 v = src[i];
            if (qb) {
                const float4 b = qb[i];
                v.x += b.x, v.y += b.y, v.z += b.z, v.w += b.w;
            }
            qv[4 * i] = v.x, qv[4 * i + 1] = v.y, qv[4 * i + 2] = v.z, qv[4 * i + 3] = v.w;
        }
    }
    SoftmaxState st;
#pragma unroll
    for (int i = 0; i < kDimsPerLane; ++i) st.acc[i] = 0.0f;

    for (uint32_t k0 = 0; k0 < length; k0 += kKeysPerChunk) {
        const uint32_t count = min((uint32_t)kKeysPerChunk, length - k0);
        __syncthreads();
        // Every load is unconditional (rows past the window repeat its last
        // row and are never read back), so all of them are in flight at once.
#pragma unroll 4
        for (int idx = threadIdx.x; idx < kKeysPerChunk * (HD / 4); idx += 64 * kWaves) {
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
        // This wavefront's share of the chunk's keys: [lo, hi).
        const uint32_t lo = count * wave / kWaves, hi = count * (wave + 1) / kWaves;
        uint32_t j = lo;
        for (; j + 1 < hi; j += 2) {
            const float d0 = slice_dot(qv, ks + j * kRow + slice);
            const float d1 = slice_dot(qv, ks + (j + 1) * kRow + slice);
            const float s0 = dev::group_sum<G>(d0) * a.scaling;
            const float s1 = dev::group_sum<G>(d1) * a.scaling;
            softmax_fold<true>(st, s0, s1, vs + j * kRow + slice, vs + (j + 1) * kRow + slice);
        }
        if (j < hi) {
            const float s0 = dev::group_sum<G>(slice_dot(qv, ks + j * kRow + slice)) * a.scaling;
            softmax_fold<false>(st, s0, 0.0f, vs + j * kRow + slice, nullptr);
        }
    }

    // Merge the wavefronts' states: wavefront w finishes dimensions
    // [4w, 4w + 4) of every lane's slice.
    __syncthreads();
    float *records = reinterpret_cast<float *>(lds);
    {
        float4 *mine = reinterpret_cast<float4 *>(records + (wave * 64 + lane) * kState);
        mine[0] = make_float4(st.max, st.sum, 0.0f, 0.0f);
#pragma unroll
        for (int i = 0; i < kDimsPerLane / 4; ++i)
            mine[1 + i] = make_float4(st.acc[4 * i], st.acc[4 * i + 1], st.acc[4 * i + 2], st.acc[4 * i + 3]);
    }
    __syncthreads();
    if (!valid) return;
    float top = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) top = fmaxf(top, records[(w * 64 + lane) * kState]);
    float total = 0.0f;
    float4 merged = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        const float *rec = records + (w * 64 + lane) * kState;
        const float weight = expf(rec[0] - top);  // 0 for a wavefront that saw no keys
        total += rec[1] * weight;
        const float4 part = reinterpret_cast<const float4 *>(rec + 4)[wave];
        merged.x += part.x * weight, merged.y += part.y * weight;
        merged.z += part.z * weight, merged.w += part.w * weight;
    }
    const float inverse = 1.0f / total;
    float4 *dst = reinterpret_cast<float4 *>(a.out + (size_t)(start + query) * a.out_stride + column + slice);
    dst[wave] = make_float4(merged.x * inverse, merged.y * inverse, merged.z * inverse, merged.w * inverse);
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
    switch (a.head_dim) {
    case 32: {
        const dim3 grid((longest + AudioTile<32>::queries - 1) / AudioTile<32>::queries, windows, a.heads);
        audio_attention_kernel<32><<<grid, 64 * kWaves, 0, s>>>(a);
        break;
    }
    case 64: {
        const dim3 grid((longest + AudioTile<64>::queries - 1) / AudioTile<64>::queries, windows, a.heads);
        audio_attention_kernel<64><<<grid, 64 * kWaves, 0, s>>>(a);
        break;
    }
    case 128: {
        const dim3 grid((longest + AudioTile<128>::queries - 1) / AudioTile<128>::queries, windows, a.heads);
        audio_attention_kernel<128><<<grid, 64 * kWaves, 0, s>>>(a);
        break;
    }
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace qwh
