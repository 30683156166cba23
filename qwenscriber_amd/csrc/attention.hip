// Grouped-query decode attention over the q8 key/value cache
// (kernels.zig:697-767 decodeAttentionStepQ8) and the q8 cache append
// (decoder.zig:68-106 appendCacheRow).
//
// The reference scores every cached position, takes a three-pass softmax and
// accumulates the dequantized values. Here the positions are split across
// workgroups (flash decoding): each workgroup streams one key/value head's
// codes for a range of positions once, for all query heads that share it, and
// keeps an online softmax (running max, running sum, rescaled accumulator).
// A second kernel merges the per-range partial states in a fixed order, so
// the result is deterministic. Position count is unbounded (the WGSL kernel's
// 4096-position cap, decode_attention_q8.wgsl:56, does not apply).
//
// Lane mapping: a head row of D codes is D/16 lanes of 16 bytes ("lane
// group"); a wavefront scores 64/(D/16) positions per load. Each lane holds
// its 16 query values for every head of the group in registers.
#include <cfloat>

#include "common.h"
#include "device.h"

namespace qwh {
namespace {

constexpr float kNeg = -1.0e30f;  // running-max sentinel: finite, so exp(kNeg - kNeg) is defined
constexpr int kBlockPositions = 4; // positions per lane group between softmax rescales
constexpr int kWaves = 4;

struct AttnKernelArgs {
    const float *query;
    const uint8_t *k_scales, *k_codes, *v_scales, *v_codes;
    const uint32_t *cached_dev;
    uint32_t cached, cached_bias;
    uint32_t heads, kv_heads;
    uint32_t chunk;      // positions per workgroup
    uint32_t splits;
    uint64_t scale_stride, code_stride;
    float scaling;
    float *partial;      // [batch][kv_heads][splits][R][D + 2]
};

__device__ __forceinline__ void unpack16(const uint4 w, float (&c)[16]) {
    const uint32_t v[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int b = 0; b < 4; ++b) c[i * 4 + b] = (float)((v[i] >> (8 * b)) & 0xffu);
    }
}

template <int D, int R>
__global__ __launch_bounds__(256) void attention_split_kernel(const AttnKernelArgs a) {
    constexpr int LPP = D / 16;              // lanes per position
    constexpr int PPW = 64 / LPP;            // positions per wave per load
    constexpr int STEP = PPW * kWaves;       // positions per workgroup per load
    constexpr int GPH = D / 64;              // scale groups per head
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int sub = lane % LPP;              // 16-byte slice of the head row
    const int group = lane / LPP;            // lane group within the wave
    const uint32_t split = blockIdx.x;
    const uint32_t kvh = blockIdx.y;
    const uint32_t b = blockIdx.z;
    const uint32_t kv_width = a.kv_heads * D;
    const uint32_t gpr = kv_width / 64;
    const uint32_t cached = a.cached_dev ? a.cached_dev[b] + a.cached_bias : a.cached;

    const uint8_t *k_scales = a.k_scales + b * a.scale_stride;
    const uint8_t *v_scales = a.v_scales + b * a.scale_stride;
    const uint8_t *k_codes = a.k_codes + b * a.code_stride;
    const uint8_t *v_codes = a.v_codes + b * a.code_stride;

    // Query slice: heads kvh*R .. kvh*R+R-1, dims sub*16 .. +16.
    float q[R][16];
    float qsum[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float4 *src = reinterpret_cast<const float4 *>(
            a.query + ((size_t)b * a.heads + kvh * R + r) * D + sub * 16);
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = src[i];
            q[r][i * 4 + 0] = v.x; q[r][i * 4 + 1] = v.y; q[r][i * 4 + 2] = v.z; q[r][i * 4 + 3] = v.w;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) s += q[r][i];
        qsum[r] = 128.0f * s;
    }

    float m[R], l[R], acc[R][16];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        m[r] = kNeg;
        l[r] = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[r][i] = 0.0f;
    }

    const uint32_t begin = split * a.chunk;
    uint32_t end = begin + a.chunk;
    if (end > cached) end = cached;
    const uint32_t scale_col = kvh * GPH + sub / 4;   // group of this lane's slice
    const uint32_t code_col = kvh * D + sub * 16;

    for (uint32_t base = begin; base < end; base += STEP * kBlockPositions) {
        uint4 kc[kBlockPositions], vc[kBlockPositions];
        float ks[kBlockPositions], vs[kBlockPositions];
        bool valid[kBlockPositions];
#pragma unroll
        for (int nb = 0; nb < kBlockPositions; ++nb) {
            const uint32_t p = base + nb * STEP + wave * PPW + group;
            valid[nb] = p < end;
            if (valid[nb]) {
                kc[nb] = *reinterpret_cast<const uint4 *>(k_codes + (size_t)p * kv_width + code_col);
                vc[nb] = *reinterpret_cast<const uint4 *>(v_codes + (size_t)p * kv_width + code_col);
                const uint16_t *kss = reinterpret_cast<const uint16_t *>(k_scales);
                const uint16_t *vss = reinterpret_cast<const uint16_t *>(v_scales);
                ks[nb] = dev::f16_bits_to_f32(kss[(size_t)p * gpr + scale_col]);
                vs[nb] = dev::f16_bits_to_f32(vss[(size_t)p * gpr + scale_col]);
            } else {
                kc[nb] = make_uint4(0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u);
                vc[nb] = kc[nb];
                ks[nb] = 0.0f;
                vs[nb] = 0.0f;
            }
        }
        // Scores: sum_i (u_i - 128) q_i = sum_i u_i q_i - 128 sum_i q_i, per
        // 16-value slice, times the slice's group scale, summed over the LPP
        // lanes of the position, times 1/sqrt(D).
        float score[kBlockPositions][R];
#pragma unroll
        for (int nb = 0; nb < kBlockPositions; ++nb) {
            float c[16];
            unpack16(kc[nb], c);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float dot = 0.0f;
#pragma unroll
                for (int i = 0; i < 16; ++i) dot = fmaf(c[i], q[r][i], dot);
                float part = (dot - qsum[r]) * ks[nb];
#pragma unroll
                for (int mask = 1; mask < LPP; mask <<= 1) part += __shfl_xor(part, mask, 64);
                score[nb][r] = valid[nb] ? part * a.scaling : kNeg;
            }
        }
        // Online softmax over the block.
        float w[kBlockPositions][R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float bm = score[0][r];
#pragma unroll
            for (int nb = 1; nb < kBlockPositions; ++nb) bm = fmaxf(bm, score[nb][r]);
            const float m_new = fmaxf(m[r], bm);
            const float alpha = expf(m[r] - m_new);
            float sum = 0.0f;
#pragma unroll
            for (int nb = 0; nb < kBlockPositions; ++nb) {
                w[nb][r] = valid[nb] ? expf(score[nb][r] - m_new) : 0.0f;
                sum += w[nb][r];
            }
            l[r] = l[r] * alpha + sum;
            m[r] = m_new;
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[r][i] *= alpha;
        }
        // Values: acc += (p * scale) * (u - 128).
#pragma unroll
        for (int nb = 0; nb < kBlockPositions; ++nb) {
            float c[16];
            unpack16(vc[nb], c);
#pragma unroll
            for (int i = 0; i < 16; ++i) c[i] -= 128.0f;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float wv = w[nb][r] * vs[nb];
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[r][i] = fmaf(wv, c[i], acc[r][i]);
            }
        }
    }

    // Merge the lane groups of this wave (lanes l and l ^ (k * LPP) hold the
    // same slice for different positions).
#pragma unroll
    for (int mask = LPP; mask < 64; mask <<= 1) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float m_o = __shfl_xor(m[r], mask, 64);
            const float l_o = __shfl_xor(l[r], mask, 64);
            const float m_new = fmaxf(m[r], m_o);
            const float a_self = expf(m[r] - m_new);
            const float a_other = expf(m_o - m_new);
            l[r] = l[r] * a_self + l_o * a_other;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float o = __shfl_xor(acc[r][i], mask, 64);
                acc[r][i] = acc[r][i] * a_self + o * a_other;
            }
            m[r] = m_new;
        }
    }

    // Merge the waves through LDS, in wave order.
    __shared__ float lds_acc[kWaves][R][D];
    __shared__ float lds_ml[kWaves][R][2];
    if (group == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int i = 0; i < 16; ++i) lds_acc[wave][r][sub * 16 + i] = acc[r][i];
            if (sub == 0) {
                lds_ml[wave][r][0] = m[r];
                lds_ml[wave][r][1] = l[r];
            }
        }
    }
    __syncthreads();
    float *out = a.partial + (((size_t)b * a.kv_heads + kvh) * a.splits + split) * R * (D + 2);
    for (int idx = threadIdx.x; idx < R * D; idx += blockDim.x) {
        const int r = idx / D;
        const int d = idx % D;
        float M = lds_ml[0][r][0];
#pragma unroll
        for (int w2 = 1; w2 < kWaves; ++w2) M = fmaxf(M, lds_ml[w2][r][0]);
        float L = 0.0f, A = 0.0f;
#pragma unroll
        for (int w2 = 0; w2 < kWaves; ++w2) {
            const float f = expf(lds_ml[w2][r][0] - M);
            L += lds_ml[w2][r][1] * f;
            A += lds_acc[w2][r][d] * f;
        }
        out[r * (D + 2) + 2 + d] = A;
        if (d == 0) {
            out[r * (D + 2) + 0] = M;
            out[r * (D + 2) + 1] = L;
        }
    }
}

// out[b][h][d] = sum_s e^{m_s - M} acc_s[d] / sum_s e^{m_s - M} l_s, splits in order.
template <int D, int R>
__global__ void attention_combine_kernel(const float *partial, uint32_t kv_heads, uint32_t splits,
                                         float *out) {
    const uint32_t b = blockIdx.y;
    const uint32_t h = blockIdx.x;
    const uint32_t kvh = h / R;
    const uint32_t r = h % R;
    const float *base = partial + ((size_t)b * kv_heads + kvh) * splits * R * (D + 2) + r * (D + 2);
    const size_t stride = (size_t)R * (D + 2);
    for (int d = threadIdx.x; d < D; d += blockDim.x) {
        float M = kNeg;
        for (uint32_t s = 0; s < splits; ++s) M = fmaxf(M, base[s * stride]);
        float L = 0.0f, A = 0.0f;
        for (uint32_t s = 0; s < splits; ++s) {
            const float f = expf(base[s * stride] - M);
            L += base[s * stride + 1] * f;
            A += base[s * stride + 2 + d] * f;
        }
        out[((size_t)b * kv_heads * R + h) * D + d] = A / L;
    }
}

// decoder.zig:94-105: quantizeRow(.q8) of one key row and one value row into
// row `position`. One wavefront per group; waves [0, gpr) take the key.
__global__ __launch_bounds__(256) void kv_append_kernel(const float *key, const float *value,
                                                        uint32_t kv_width, uint32_t position,
                                                        uint8_t *k_scales, uint8_t *k_codes,
                                                        uint8_t *v_scales, uint8_t *v_codes) {
    const uint32_t gpr = kv_width / 64;
    const uint32_t wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (wave >= 2 * gpr) return;
    const bool is_key = wave < gpr;
    const uint32_t g = is_key ? wave : wave - gpr;
    const float v = (is_key ? key : value)[g * 64 + lane];
    uint8_t *scales = is_key ? k_scales : v_scales;
    uint8_t *codes = is_key ? k_codes : v_codes;
    const float amax = dev::wave_max(fabsf(v));
    const uint16_t bits = dev::f32_to_f16_bits(__fdiv_rn(amax, 128.0f));
    const float stored = dev::f16_bits_to_f32(bits);
    codes[(size_t)position * kv_width + g * 64 + lane] =
        (uint8_t)(dev::quantize_one(v, stored, -128, 127) + 128);
    if (lane == 0) reinterpret_cast<uint16_t *>(scales)[(size_t)position * gpr + g] = bits;
}

void attention_shape(int cus, const AttentionArgs &a, uint32_t &chunk, uint32_t &splits) {
    // Positions per workgroup: a multiple of one full block (STEP * 4); enough
    // workgroups to fill the device about twice.
    const uint32_t lpp = a.head_dim / 16;
    const uint32_t step = (64 / lpp) * kWaves * kBlockPositions;
    const uint32_t target = (uint32_t)(cus > 0 ? cus : 256) * 2;
    const uint32_t pairs = a.batch * a.kv_heads;
    uint32_t want_splits = (target + pairs - 1) / pairs;
    if (want_splits < 1) want_splits = 1;
    uint32_t per = (a.capacity + want_splits - 1) / want_splits;
    chunk = ((per + step - 1) / step) * step;
    if (chunk < step) chunk = step;
    splits = (a.capacity + chunk - 1) / chunk;
    if (splits < 1) splits = 1;
}

}  // namespace

size_t attention_scratch_bytes(int cus, const AttentionArgs &a) {
    uint32_t chunk, splits;
    attention_shape(cus, a, chunk, splits);
    const uint32_t R = a.heads / a.kv_heads;
    return (size_t)a.batch * a.kv_heads * splits * R * (a.head_dim + 2) * sizeof(float) + 256;
}

#define QWH_ATTN_CASE(D_, R_)                                                                   \
    if (a.head_dim == D_ && R == R_) {                                                          \
        attention_split_kernel<D_, R_><<<dim3(splits, a.kv_heads, a.batch), 256, 0, s>>>(k);    \
        attention_combine_kernel<D_, R_><<<dim3(a.heads, a.batch), D_, 0, s>>>(                 \
            k.partial, a.kv_heads, splits, a.out);                                              \
        return hipGetLastError();                                                               \
    }

hipError_t launch_decode_attention_q8(hipStream_t s, int cus, const AttentionArgs &a, void *scratch) {
    uint32_t chunk, splits;
    attention_shape(cus, a, chunk, splits);
    const uint32_t R = a.heads / a.kv_heads;
    AttnKernelArgs k{};
    k.query = a.query;
    k.k_scales = a.k_scales;
    k.k_codes = a.k_codes;
    k.v_scales = a.v_scales;
    k.v_codes = a.v_codes;
    k.cached_dev = a.cached_dev;
    k.cached = a.cached;
    k.cached_bias = a.cached_bias;
    k.heads = a.heads;
    k.kv_heads = a.kv_heads;
    k.chunk = chunk;
    k.splits = splits;
    k.scale_stride = a.scale_stride;
    k.code_stride = a.code_stride;
    k.scaling = 1.0f / sqrtf((float)a.head_dim);  // kernels.zig:727
    k.partial = static_cast<float *>(scratch);
    QWH_ATTN_CASE(64, 1)
    QWH_ATTN_CASE(64, 2)
    QWH_ATTN_CASE(64, 4)
    QWH_ATTN_CASE(128, 1)
    QWH_ATTN_CASE(128, 2)
    QWH_ATTN_CASE(128, 4)
    QWH_ATTN_CASE(128, 8)
    QWH_ATTN_CASE(256, 1)
    QWH_ATTN_CASE(256, 2)
    return hipErrorNotSupported;
}

hipError_t launch_kv_append_q8(hipStream_t s, const float *key, const float *value, uint32_t kv_width,
                               uint32_t position, uint8_t *k_scales, uint8_t *k_codes,
                               uint8_t *v_scales, uint8_t *v_codes) {
    const uint32_t waves = 2 * (kv_width / 64);
    kv_append_kernel<<<(waves + 3) / 4, 256, 0, s>>>(key, value, kv_width, position, k_scales, k_codes,
                                                     v_scales, v_codes);
    return hipGetLastError();
}

}  // namespace qwh
