// Grouped-query decode attention over the q8 key/value cache
// (kernels.zig:697-767 decodeAttentionStepQ8) and the q8 cache append
// (decoder.zig:68-106 appendCacheRow).
//
// The reference scores every cached position, takes a three-pass softmax and
// accumulates the dequantized values. Here the positions are split across
// workgroups (flash decoding): each workgroup streams one key/value head's
// codes for a range of positions once, for all query heads that share it, and
// keeps an online softmax (running max, running sum, rescaled accumulator).
// Every workgroup writes its partial state; a second kernel merges the
// partials of all ranges in range order, so the result is deterministic.
// (Merging in the last workgroup to finish needs device-scope fences, which
// write back and invalidate the L2 of every die and measured slower.)
// Position count is unbounded (the WGSL kernel's 4096-position cap,
// decode_attention_q8.wgsl:56, does not apply).
//
// The decoder form also does the work decoder.zig:180-216 does between the
// q/k/v projection and the attention: per-head RMSNorm of q and k, RoPE at the
// new position, and the q8 append of the new key and value rows. Every
// workgroup normalizes and rotates its own query heads; the workgroup whose
// range holds the new position also quantizes the new key/value rows, stores
// them in the cache, and attends to them from registers.
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
constexpr uint32_t kMaxSplits = 512;

struct AttnKernelArgs {
    const float *query;  // row of sequence b at query + b * query_stride; head h at h * D
    uint32_t query_stride;
    uint8_t *k_scales, *k_codes, *v_scales, *v_codes;
    const uint32_t *cached_dev;
    uint32_t cached, cached_bias;
    uint32_t heads, kv_heads;
    uint32_t chunk;      // positions per workgroup
    uint32_t splits;
    uint64_t scale_stride, code_stride;
    float scaling;
    float *partial;      // [batch][kv_heads][splits] records of R*D + 4*R floats
    float *out;          // [batch][heads][D]
    // Decoder form.
    const float *q_norm, *k_norm, *rope_cos, *rope_sin;
    float eps;
};

__device__ __forceinline__ void unpack16(const uint4 w, float (&c)[16]) {
    const uint32_t v[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int b = 0; b < 4; ++b) c[i * 4 + b] = (float)((v[i] >> (8 * b)) & 0xffu);
    }
}

template <int LPP>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int mask = 1; mask < LPP; mask <<= 1) v += __shfl_xor(v, mask, 64);
    return v;
}

// math.rmsNormInPlace (math.zig:120-130) of one head row spread over the LPP
// lanes of a lane group (16 values per lane), then rotate_half RoPE
// (kernels.zig:495-527) with the tables' row for `pos`: the partner of
// dimension d < D/2 is d + D/2, held by lane sub ^ LPP/2.
template <int D>
__device__ __forceinline__ void norm_rope16(float (&x)[16], const float *weight, const float *cos_row,
                                            const float *sin_row, int sub, float eps) {
    constexpr int LPP = D / 16;
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) ss = __fadd_rn(ss, __fmul_rn(x[i], x[i]));
    ss = group_sum<LPP>(ss);
    const float inverse_rms = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)D), eps)));
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = __fmul_rn(__fmul_rn(x[i], inverse_rms), weight[sub * 16 + i]);
    const bool first = sub < LPP / 2;
    const int j0 = (sub % (LPP / 2)) * 16;
    float y[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float partner = __shfl_xor(x[i], LPP / 2, 64);
        const float c = cos_row[j0 + i];
        const float s = sin_row[j0 + i];
        y[i] = first ? __fsub_rn(__fmul_rn(x[i], c), __fmul_rn(partner, s))
                     : __fadd_rn(__fmul_rn(x[i], c), __fmul_rn(partner, s));
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = y[i];
}

// quantizeRow(.q8) (quant.zig:197-288) of a head row: the 64-value groups are
// 4 consecutive lanes of a lane group. Returns this lane's 16 codes packed in
// byte order, and its group's stored scale (bits and value).
__device__ __forceinline__ uint4 quantize16(const float (&x)[16], uint16_t &bits, float &stored) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(x[i]));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    bits = dev::f32_to_f16_bits(__fdiv_rn(amax, 128.0f));
    stored = dev::f16_bits_to_f32(bits);
    uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 16; ++i)
        w[i / 4] |= (uint32_t)(dev::quantize_one(x[i], stored, -128, 127) + 128) << (8 * (i % 4));
    return make_uint4(w[0], w[1], w[2], w[3]);
}

template <int R>
struct SoftmaxState {
    float m[R], l[R], acc[R][16];
};

// One block of NB positions per lane group: scores against the lane's query
// slices, online-softmax update, value accumulation.
template <int D, int R, int NB>
__device__ __forceinline__ void attend(SoftmaxState<R> &st, const float (&q)[R][16], const float (&qsum)[R],
                                       const uint4 (&kc)[NB], const uint4 (&vc)[NB], const float (&ks)[NB],
                                       const float (&vs)[NB], const bool (&valid)[NB], float scaling) {
    constexpr int LPP = D / 16;
    // Scores: sum_i (u_i - 128) q_i = sum_i u_i q_i - 128 sum_i q_i, per
    // 16-value slice, times the slice's group scale, summed over the LPP
    // lanes of the position, times 1/sqrt(D).
    float score[NB][R];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        float c[16];
        unpack16(kc[nb], c);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float dot = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) dot = fmaf(c[i], q[r][i], dot);
            const float part = group_sum<LPP>((dot - qsum[r]) * ks[nb]);
            score[nb][r] = valid[nb] ? part * scaling : kNeg;
        }
    }
    float w[NB][R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float bm = score[0][r];
#pragma unroll
        for (int nb = 1; nb < NB; ++nb) bm = fmaxf(bm, score[nb][r]);
        const float m_new = fmaxf(st.m[r], bm);
        const float alpha = expf(st.m[r] - m_new);
        float sum = 0.0f;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            w[nb][r] = valid[nb] ? expf(score[nb][r] - m_new) : 0.0f;
            sum += w[nb][r];
        }
        st.l[r] = st.l[r] * alpha + sum;
        st.m[r] = m_new;
#pragma unroll
        for (int i = 0; i < 16; ++i) st.acc[r][i] *= alpha;
    }
    // Values: acc += (p * scale) * (u - 128), the code offset taken exactly.
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        float c[16];
        unpack16(vc[nb], c);
#pragma unroll
        for (int i = 0; i < 16; ++i) c[i] -= 128.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float wv = w[nb][r] * vs[nb];
#pragma unroll
            for (int i = 0; i < 16; ++i) st.acc[r][i] = fmaf(wv, c[i], st.acc[r][i]);
        }
    }
}

// out[h][d] = sum_s e^{m_s - M} acc_s[d] / sum_s e^{m_s - M} l_s over the
// ranges that hold positions, in range order, for the R heads of kv head
// `kvh`. Thread t takes four dimensions of one head (column t % COLS) for the
// ranges congruent to t / COLS; the SL partial merges are then combined in
// order.
template <int D, int R>
__device__ __forceinline__ void merge_ranges(const AttnKernelArgs &a, uint32_t b, uint32_t kvh, uint32_t cached) {
    constexpr int REC = R * D + 4 * R;
    constexpr int COLS = R * D / 4;
    static_assert(COLS <= 256, "one float4 column per thread");
    constexpr int SL = 256 / COLS;
    const uint32_t used = (cached + a.chunk - 1) / a.chunk < a.splits ? (cached + a.chunk - 1) / a.chunk : a.splits;
    const int t = threadIdx.x;
    const int col = t % COLS;
    const int j = t / COLS;
    const int r = col / (D / 4);
    const int d4 = col % (D / 4);
    float M = kNeg, L = 0.0f;
    float4 A = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float *recs = a.partial + ((size_t)b * a.kv_heads + kvh) * a.splits * REC;
    if (j < SL) {
        for (uint32_t s = j; s < used; s += SL) {
            const float *rec = recs + (size_t)s * REC;
            const float m = rec[R * D + 4 * r];
            const float l = rec[R * D + 4 * r + 1];
            const float4 v = *reinterpret_cast<const float4 *>(rec + r * D + 4 * d4);
            const float m_new = fmaxf(M, m);
            const float fa = expf(M - m_new);
            const float fb = expf(m - m_new);
            L = L * fa + l * fb;
            A.x = A.x * fa + v.x * fb;
            A.y = A.y * fa + v.y * fb;
            A.z = A.z * fa + v.z * fb;
            A.w = A.w * fa + v.w * fb;
            M = m_new;
        }
    }
    __shared__ float lds_m[256], lds_l[256];
    __shared__ float4 lds_a[256];
    lds_m[t] = M;
    lds_l[t] = L;
    lds_a[t] = A;
    __syncthreads();
    if (t < COLS) {
        for (int k = 1; k < SL; ++k) {
            const float m = lds_m[k * COLS + col];
            const float l = lds_l[k * COLS + col];
            const float4 v = lds_a[k * COLS + col];
            const float m_new = fmaxf(M, m);
            const float fa = expf(M - m_new);
            const float fb = expf(m - m_new);
            L = L * fa + l * fb;
            A.x = A.x * fa + v.x * fb;
            A.y = A.y * fa + v.y * fb;
            A.z = A.z * fa + v.z * fb;
            A.w = A.w * fa + v.w * fb;
            M = m_new;
        }
        const float inv = 1.0f / L;
        float4 o = make_float4(A.x * inv, A.y * inv, A.z * inv, A.w * inv);
        *reinterpret_cast<float4 *>(a.out + ((size_t)b * a.heads + kvh * R + r) * D + 4 * d4) = o;
    }
}

template <int D, int R, bool Decoder>
__global__ __launch_bounds__(256) void attention_kernel(const AttnKernelArgs a) {
    constexpr int LPP = D / 16;              // lanes per position
    constexpr int PPW = 64 / LPP;            // positions per wave per load
    constexpr int STEP = PPW * kWaves;       // positions per workgroup per load
    constexpr int GPH = D / 64;              // scale groups per head
    constexpr int REC = R * D + 4 * R;       // floats per partial record
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
    const uint32_t begin = split * a.chunk;
    uint32_t end = begin + a.chunk;
    if (end > cached) end = cached;

    __shared__ float lds_acc[kWaves][R][D];
    __shared__ float lds_ml[kWaves][R][2];

    if (begin < cached) {
        const uint16_t *k_scales = reinterpret_cast<const uint16_t *>(a.k_scales + b * a.scale_stride);
        const uint16_t *v_scales = reinterpret_cast<const uint16_t *>(a.v_scales + b * a.scale_stride);
        const uint8_t *k_codes = a.k_codes + b * a.code_stride;
        const uint8_t *v_codes = a.v_codes + b * a.code_stride;
        const uint32_t scale_col = kvh * GPH + sub / 4;   // group of this lane's slice
        const uint32_t code_col = kvh * D + sub * 16;
        // The decoder form's new row (position cached - 1) is attended from
        // registers by the workgroup that holds it, so the loop stops short.
        const uint32_t newest = cached - 1;
        const bool owner = Decoder && end == cached;
        const uint32_t loop_end = owner ? newest : end;

        // Query slices: heads kvh*R .. kvh*R+R-1, dims sub*16 .. +16.
        const float *row = a.query + (size_t)b * a.query_stride;
        float q[R][16];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float4 *src = reinterpret_cast<const float4 *>(row + (kvh * R + r) * D + sub * 16);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 v = src[i];
                q[r][i * 4 + 0] = v.x; q[r][i * 4 + 1] = v.y; q[r][i * 4 + 2] = v.z; q[r][i * 4 + 3] = v.w;
            }
        }
        if (Decoder) {
            const float *cos_row = a.rope_cos + (size_t)newest * (D / 2);
            const float *sin_row = a.rope_sin + (size_t)newest * (D / 2);
#pragma unroll
            for (int r = 0; r < R; ++r) norm_rope16<D>(q[r], a.q_norm, cos_row, sin_row, sub, a.eps);
        }
        float qsum[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) s += q[r][i];
            qsum[r] = 128.0f * s;
        }

        SoftmaxState<R> st;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            st.m[r] = kNeg;
            st.l[r] = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) st.acc[r][i] = 0.0f;
        }

        for (uint32_t base = begin; base < loop_end; base += STEP * kBlockPositions) {
            uint4 kc[kBlockPositions], vc[kBlockPositions];
            float ks[kBlockPositions], vs[kBlockPositions];
            bool valid[kBlockPositions];
#pragma unroll
            for (int nb = 0; nb < kBlockPositions; ++nb) {
                const uint32_t p = base + nb * STEP + wave * PPW + group;
                valid[nb] = p < loop_end;
                if (valid[nb]) {
                    kc[nb] = *reinterpret_cast<const uint4 *>(k_codes + (size_t)p * kv_width + code_col);
                    vc[nb] = *reinterpret_cast<const uint4 *>(v_codes + (size_t)p * kv_width + code_col);
                    ks[nb] = dev::f16_bits_to_f32(k_scales[(size_t)p * gpr + scale_col]);
                    vs[nb] = dev::f16_bits_to_f32(v_scales[(size_t)p * gpr + scale_col]);
                } else {
                    kc[nb] = make_uint4(0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u);
                    vc[nb] = kc[nb];
                    ks[nb] = 0.0f;
                    vs[nb] = 0.0f;
                }
            }
            attend<D, R, kBlockPositions>(st, q, qsum, kc, vc, ks, vs, valid, a.scaling);
        }

        if (owner) {
            // decoder.zig:180-216 for the kv head of this workgroup: RMSNorm
            // and RoPE of the key, then the q8 append of key and value.
            const float *key = row + a.heads * D + kvh * D + sub * 16;
            const float *value = row + a.heads * D + kv_width + kvh * D + sub * 16;
            float kx[16], vx[16];
#pragma unroll
            for (int i = 0; i < 16; i += 4) {
                const float4 kv4 = *reinterpret_cast<const float4 *>(key + i);
                const float4 vv4 = *reinterpret_cast<const float4 *>(value + i);
                kx[i] = kv4.x; kx[i + 1] = kv4.y; kx[i + 2] = kv4.z; kx[i + 3] = kv4.w;
                vx[i] = vv4.x; vx[i + 1] = vv4.y; vx[i + 2] = vv4.z; vx[i + 3] = vv4.w;
            }
            norm_rope16<D>(kx, a.k_norm, a.rope_cos + (size_t)newest * (D / 2), a.rope_sin + (size_t)newest * (D / 2),
                           sub, a.eps);
            uint16_t kbits, vbits;
            uint4 kc[1], vc[1];
            float ks[1], vs[1];
            kc[0] = quantize16(kx, kbits, ks[0]);
            vc[0] = quantize16(vx, vbits, vs[0]);
            if (wave == 0 && group == 0) {
                *reinterpret_cast<uint4 *>(a.k_codes + b * a.code_stride + (size_t)newest * kv_width + code_col) = kc[0];
                *reinterpret_cast<uint4 *>(a.v_codes + b * a.code_stride + (size_t)newest * kv_width + code_col) = vc[0];
                if (sub % 4 == 0) {
                    reinterpret_cast<uint16_t *>(a.k_scales + b * a.scale_stride)[(size_t)newest * gpr + scale_col] = kbits;
                    reinterpret_cast<uint16_t *>(a.v_scales + b * a.scale_stride)[(size_t)newest * gpr + scale_col] = vbits;
                }
            }
            const bool valid[1] = {wave == 0 && group == 0};
            attend<D, R, 1>(st, q, qsum, kc, vc, ks, vs, valid, a.scaling);
        }

        // Merge the lane groups of this wave (lanes l and l ^ (k * LPP) hold
        // the same slice for different positions).
#pragma unroll
        for (int mask = LPP; mask < 64; mask <<= 1) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float m_o = __shfl_xor(st.m[r], mask, 64);
                const float l_o = __shfl_xor(st.l[r], mask, 64);
                const float m_new = fmaxf(st.m[r], m_o);
                const float a_self = expf(st.m[r] - m_new);
                const float a_other = expf(m_o - m_new);
                st.l[r] = st.l[r] * a_self + l_o * a_other;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const float o = __shfl_xor(st.acc[r][i], mask, 64);
                    st.acc[r][i] = st.acc[r][i] * a_self + o * a_other;
                }
                st.m[r] = m_new;
            }
        }
        if (group == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
#pragma unroll
                for (int i = 0; i < 16; ++i) lds_acc[wave][r][sub * 16 + i] = st.acc[r][i];
                if (sub == 0) {
                    lds_ml[wave][r][0] = st.m[r];
                    lds_ml[wave][r][1] = st.l[r];
                }
            }
        }
        __syncthreads();
        // Merge the waves in wave order into this range's record.
        float *rec = a.partial + (((size_t)b * a.kv_heads + kvh) * a.splits + split) * REC;
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
            rec[idx] = A;
            if (d == 0) {
                rec[R * D + 4 * r + 0] = M;
                rec[R * D + 4 * r + 1] = L;
            }
        }
    }

}

template <int D, int R>
__global__ __launch_bounds__(256) void attention_combine_kernel(const AttnKernelArgs a) {
    const uint32_t kvh = blockIdx.x;
    const uint32_t b = blockIdx.y;
    const uint32_t cached = a.cached_dev ? a.cached_dev[b] + a.cached_bias : a.cached;
    merge_ranges<D, R>(a, b, kvh, cached);
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
    // workgroups to fill the device about twice, at most kMaxSplits ranges.
    const uint32_t lpp = a.head_dim / 16;
    const uint32_t step = (64 / lpp) * kWaves * kBlockPositions;
    const uint32_t target = (uint32_t)(cus > 0 ? cus : 256) * 2;
    const uint32_t pairs = a.batch * a.kv_heads;
    uint32_t want_splits = (target + pairs - 1) / pairs;
    if (want_splits < 1) want_splits = 1;
    if (want_splits > kMaxSplits) want_splits = kMaxSplits;
    const uint32_t per = (a.capacity + want_splits - 1) / want_splits;
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
    return (size_t)a.batch * a.kv_heads * splits * (R * a.head_dim + 4 * R) * sizeof(float) + 256;
}

bool attention_supported(uint32_t head_dim, uint32_t ratio) {
    return (head_dim == 64 && (ratio == 1 || ratio == 2 || ratio == 4)) ||
           (head_dim == 128 && (ratio == 1 || ratio == 2 || ratio == 4 || ratio == 8)) ||
           (head_dim == 256 && (ratio == 1 || ratio == 2));
}

#define QWH_ATTN_CASE(D_, R_)                                                                       \
    if (a.head_dim == D_ && R == R_) {                                                              \
        if (decoder)                                                                                \
            attention_kernel<D_, R_, true><<<dim3(splits, a.kv_heads, a.batch), 256, 0, s>>>(k);    \
        else                                                                                        \
            attention_kernel<D_, R_, false><<<dim3(splits, a.kv_heads, a.batch), 256, 0, s>>>(k);   \
        attention_combine_kernel<D_, R_><<<dim3(a.kv_heads, a.batch), 256, 0, s>>>(k);              \
        return hipGetLastError();                                                                   \
    }

hipError_t launch_decode_attention_q8(hipStream_t s, int cus, const AttentionArgs &a, void *scratch) {
    uint32_t chunk, splits;
    attention_shape(cus, a, chunk, splits);
    const uint32_t R = a.heads / a.kv_heads;
    const bool decoder = a.q_norm != nullptr;
    AttnKernelArgs k{};
    k.query = a.query;
    k.query_stride = a.query_stride ? a.query_stride : a.heads * a.head_dim;
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
    k.out = a.out;
    k.q_norm = a.q_norm;
    k.k_norm = a.k_norm;
    k.rope_cos = a.rope_cos;
    k.rope_sin = a.rope_sin;
    k.eps = a.eps;
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
