// Batch-1 (and small-batch) decode GEMV over the reference's packed planes.
//
// kernels.zig:118-158 linearQuantized with tokens small. The reference
// dequantizes a row into f32 scratch and dots it with the activations; here a
// row's codes are streamed once from HBM with 128-bit loads and multiplied in
// registers without ever forming a dequantized weight:
//
//   q4: the activations are written as signed hex digit planes (device.h);
//       each 16-byte load of codes holds 32 weights, XOR 0x8 turns every
//       biased nibble u into the signed code u - 8, and a Horner chain of
//       v_dot8_i32_i4 over the six digit planes gives the exact integer dot
//       product, converted once to f32 and scaled by the group's f16 scale
//       times the chunk's power-of-two activation multiplier.
//   q8: each 16-byte load holds 16 codes, converted to f32 (exact) and
//       multiplied with f32 activations.
//
// Lane mapping: a row of K codes is T = K/32 (q4) or K/16 (q8) 16-byte
// slices. L = gcd(T, 64) lanes share a row, so a wavefront covers RG = 64/L
// consecutive rows (a "row group") and each lane always handles the same S =
// T/L slices of its row: its activation operands stay in registers for the
// whole kernel while the wave walks row groups. Units of U row groups are
// dealt out grid-stride (wave w takes units w, w + waves, ...; the grid holds
// no more blocks than can be resident), so the waves together stream one
// compact window of the matrix; a wave issues its next unit's 128-bit loads
// before it multiplies the current one, and reduces the U row sums of each
// row with one transposed butterfly over the row's L lanes.
//
// The q4 kernel takes its activations in one of three forms: prepared digit
// planes, or f32 values that each wavefront encodes itself -- as they are, or
// after RMSNorm (kernels.zig:274-300, decoder.zig:165-172: the statistics of
// the row are reduced over the lanes that hold it). The last two let the
// decoder step feed a GEMV straight from the previous kernel's f32 output.
// Its output is either the N row products (plus an optional residual) or,
// for a matrix whose rows alternate gate and up rows, siluMul of each pair
// (kernels.zig:233-239), so the gate/up projection hands the down projection
// its f32 input directly.
#include <cfloat>
#include <cstdlib>
#include <mutex>
#include <unordered_map>

#include "common.h"
#include "device.h"

namespace qwh {
namespace {

constexpr int kWave = 64;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// 128-bit streaming load (weights are read once per call: no reuse to keep).
__device__ __forceinline__ uint4 load_stream16(const void *p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// f16 scale `index` of a plane below 4 GiB, addressed with a 32-bit byte
// offset so the load uses the plane's scalar base.
__device__ __forceinline__ uint16_t load_scale(const uint16_t *plane, uint32_t index) {
    return *reinterpret_cast<const uint16_t *>(reinterpret_cast<const uint8_t *>(plane) + index * 2u);
}

template <int V>
struct Log2 {
    static constexpr int value = 1 + Log2<V / 2>::value;
};
template <>
struct Log2<1> {
    static constexpr int value = 0;
};

// One exchange step of the transposed reduction: the lanes with bit MASK set
// keep b and send a, the others keep a and send b; returns keep + received.
template <int MASK>
__device__ __forceinline__ float exchange(float a, float b, int lane) {
    const bool upper = (lane & MASK) != 0;
    const float send = upper ? a : b;
    const float keep = upper ? b : a;
    return keep + dev::xor_lane<MASK>(send);
}

// Sums acc[0..U) (U <= 8) over the L lanes of each row (lanes l and l ^ m
// with m < L share a row). Returns, in every lane, the total of value
// ((l % L) >> (log2 L - log2 U)) of its row.
template <int U, int L>
__device__ __forceinline__ float reduce_rows(const float (&acc)[U], int lane) {
    static_assert(U == 1 || U == 2 || U == 4 || U == 8, "U must be 1, 2, 4 or 8");
    static_assert(U <= L, "more values than lanes per row");
    constexpr int log_u = Log2<U>::value;
    float v;
    if constexpr (U == 1) {
        v = acc[0];
    } else if constexpr (U == 2) {
        v = exchange<L / 2>(acc[0], acc[1], lane);
    } else if constexpr (U == 4) {
        const float b0 = exchange<L / 2>(acc[0], acc[2], lane);
        const float b1 = exchange<L / 2>(acc[1], acc[3], lane);
        v = exchange<L / 4>(b0, b1, lane);
    } else {
        const float b0 = exchange<L / 2>(acc[0], acc[4], lane);
        const float b1 = exchange<L / 2>(acc[1], acc[5], lane);
        const float b2 = exchange<L / 2>(acc[2], acc[6], lane);
        const float b3 = exchange<L / 2>(acc[3], acc[7], lane);
        const float c0 = exchange<L / 4>(b0, b2, lane);
        const float c1 = exchange<L / 4>(b1, b3, lane);
        v = exchange<L / 8>(c0, c1, lane);
    }
    return dev::group_sum<(L >> log_u)>(v);
}

// Sum of v over the L lanes of a row.
template <int L>
__device__ __forceinline__ float row_sum(float v) {
    return dev::group_sum<L>(v);
}

// ---------------------------------------------------------------------------
// Digit planes of the activations as a separate pass (for the shapes the
// fused kernels do not cover): one thread per 8 consecutive values, four
// threads per 32-value chunk.
// Layout: words[(t * T + c) * 24 + plane * 4 + q], mult[t * T + c].
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void prep_q4_kernel(const float *x, uint32_t total8,
                                                      uint32_t *words, float *mult) {
    const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
    const bool valid = gid < total8;
    float v[8];
    if (valid) {
        const float4 a = reinterpret_cast<const float4 *>(x)[gid * 2];
        const float4 b = reinterpret_cast<const float4 *>(x)[gid * 2 + 1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = 0.0f;
    }
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) amax = fmaxf(amax, fabsf(v[k]));
    amax = fmaxf(amax, dev::xor_lane<1>(amax));
    amax = fmaxf(amax, dev::xor_lane<2>(amax));
    const int e = dev::chunk_exponent(amax);
    uint32_t planes[6];
    dev::encode_digits8(v, e, planes);
    if (valid) {
        const uint32_t chunk = gid >> 2;
        const uint32_t q = gid & 3u;
        uint32_t *dst = words + (size_t)chunk * dev::kChunkWords + q;
#pragma unroll
        for (int j = 0; j < 6; ++j) dst[j * 4] = planes[j];
        if (q == 0) mult[chunk] = __builtin_ldexpf(1.0f, e - 22);
    }
}

// Exact integer dot product of one 16-byte slice of q4 codes (32 weights)
// with its activations' digit planes: sum_k (u_k - 8) * x_int_k. Two
// independent Horner chains, planes 5..3 and planes 2..0, each step a run of
// four v_dot8_i32_i4, joined as hi * 16^3 + lo. Two chains halve the
// dependent-issue latency of one chain of 24; that latency is what the
// last units of a launch pay after their data has arrived. Every partial
// value is bounded by 32 * 8 * 2^22 = 2^30, so the int32 result is exact
// (and equal to the single-chain Horner value).
__device__ __forceinline__ int q4_slice_dot(const uint4 codes, const uint32_t (&d)[24]) {
    const int c[4] = {(int)(codes.x ^ 0x88888888u), (int)(codes.y ^ 0x88888888u), (int)(codes.z ^ 0x88888888u),
                      (int)(codes.w ^ 0x88888888u)};
    int hi = 0, lo = 0;
#pragma unroll
    for (int j = 2; j >= 0; --j) {
        if (j != 2) {
            hi = hi * 16;
            lo = lo * 16;
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            hi = __builtin_amdgcn_sdot8(c[q], (int)d[(j + 3) * 4 + q], hi, false);
            lo = __builtin_amdgcn_sdot8(c[q], (int)d[j * 4 + q], lo, false);
        }
    }
    return hi * 4096 + lo;
}

// Forms of the q4 GEMV's activations: prepared digit planes; f32 values;
// f32 values after RMSNorm; a token's embedding row (or an audio row) after
// RMSNorm (Embed: the first q | k | v projection of a decoder step).
enum class Src : int { Digits = 0, F32 = 1, RmsNorm = 2, Embed = 4 };

struct GemvQ4Args {
    const uint32_t *words;  // Digits: planes, per token T * 24 words
    const float *mult;      // Digits: per token T multipliers
    const float *x;         // F32 / RmsNorm: tokens x K
    const float *norm;      // RmsNorm: K weights
    float eps;              // RmsNorm epsilon
    const uint16_t *scales; // N * K/64
    const uint8_t *data;    // N * K/2
    float *out;             // tokens x N, or tokens x N/2 with pairs
    const float *residual;  // optional, tokens x N (may alias out); not with pairs
    uint32_t n, k, t, row_groups;
    uint32_t pairs;         // rows 2j, 2j+1 are gate_j, up_j: write silu(gate_j) * up_j
    // Embed: tokens[token]'s row of the embedding matrix (format
    // embed_format), or, where row_flags[token] is set, row `token` of
    // rows; workgroup 0 of each token also stores the row to hidden_out and
    // the RoPE table row of position pos[token] (rope_half cos, then sin) to
    // rope_now.
    const uint32_t *tokens;
    int32_t embed_format;
    const uint16_t *embed_scales;
    const uint8_t *embed_data;
    const float *rows;
    const uint32_t *row_flags;
    float *hidden_out;
    const uint32_t *pos;
    const float *rope_cos, *rope_sin;
    uint32_t rope_half;
    float *rope_now;
    // Optional argmax partials of the outputs (decoder.zig:290-301
    // argmaxLogits, no residual, no pairs): per token and workgroup the
    // largest output and its lowest row among equal maxima, at
    // [token * gridDim.x + blockIdx.x].
    float *arg_value;
    uint32_t *arg_index;
};

// The better of two (value, row) candidates of argmaxLogits: the larger
// value, the lower row among equal values; a NaN is never taken.
__device__ __forceinline__ void arg_better(float &v, uint32_t &i, float v2, uint32_t i2) {
    if (v2 > v || (v2 == v && i2 < i)) {
        v = v2;
        i = i2;
    }
}

// siluMul of one gate / up pair (math.zig:69-71: silu(g) = g / (1 + exp(-g))).
__device__ __forceinline__ float silu_mul(float g, float u) {
    return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, expf(-g))), u);
}

// One 16-byte slice of codes and its group scale.
struct Slice {
    uint4 codes;
    uint16_t scale;
};

// Activation digits of a whole row, encoded once per workgroup into LDS:
// thread t takes values 8t .. 8t+7 of each 2048-value stretch (the four
// threads of a 32-value chunk are consecutive lanes), so the block shares the
// work instead of every wavefront encoding the row for itself. K is at most
// 3 * 64 * 32 = 6144 (the fused shapes), i.e. at most 3 stretches.
constexpr int kMaxChunks = 192;
struct ActLds {
    uint32_t words[kMaxChunks * 24];
    float mult[kMaxChunks];
    float partial[4];
};

// A value no kernel writes while this one runs (a sequence's position, its
// token), read through the scalar cache: the wait for it then does not wait
// for the vector loads issued before it.
__device__ __forceinline__ uint32_t load_uniform(const uint32_t *p) {
    return *(const __attribute__((address_space(4))) uint32_t *)p;
}

// The row's values (and RMSNorm weights) this thread encodes, fetched before
// the first unit's weights are requested: the wait for them then leaves the
// weight loads in flight (loads complete in issue order). Threads past the
// row's end load its last 8 values and drop them in block_encode.
struct RowValues {
    float v[3][8];
    float w[3][8];
    uint32_t tok, audio, pos;  // Embed: the token, its row flag and position
};

// Embed: values 8 e8 .. 8 e8 + 7 of row `tok` of the embedding matrix
// (decoder.zig:346-376 embeddingRow; quant.zig:315-345 dequantizeGroup):
// f32(u - bias) times the group's scale.
__device__ __forceinline__ void embed_fetch(const GemvQ4Args &a, uint32_t tok, uint32_t e8, float (&out)[8]) {
    const uint32_t gpr = a.k >> 6;
    const float scale = dev::f16_bits_to_f32(a.embed_scales[(size_t)tok * gpr + e8 / 8]);
    if (a.embed_format == QWH_FORMAT_Q4) {
        const uint32_t w = *reinterpret_cast<const uint32_t *>(a.embed_data + (size_t)tok * (a.k / 2) + 4 * e8);
#pragma unroll
        for (int i = 0; i < 8; ++i) out[i] = __fmul_rn((float)((int)((w >> (4 * i)) & 0xfu) - 8), scale);
    } else if (a.embed_format == QWH_FORMAT_Q8) {
        const uint2 w = *reinterpret_cast<const uint2 *>(a.embed_data + (size_t)tok * a.k + 8 * e8);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t word = i < 4 ? w.x : w.y;
            out[i] = __fmul_rn((float)((int)((word >> (8 * (i & 3))) & 0xffu) - 128), scale);
        }
    } else {
        // q5: the low nibbles as q4, the fifth bit of value j in bit j % 8 of
        // byte 32 + j / 8 of the group.
        const uint8_t *g = a.embed_data + ((size_t)tok * gpr + e8 / 8) * 40;
        const uint32_t j0 = (e8 % 8) * 8;
        const uint32_t w = *reinterpret_cast<const uint32_t *>(g + j0 / 2);
        const uint32_t high = g[32 + j0 / 8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t u = ((w >> (4 * i)) & 0xfu) | (((high >> i) & 1u) << 4);
            out[i] = __fmul_rn((float)((int)u - 16), scale);
        }
    }
}

template <Src M>
__device__ __forceinline__ void block_fetch(const GemvQ4Args &a, uint32_t token, RowValues &rv) {
    const int tid = threadIdx.x;
    const uint32_t k8 = a.k / 8;
    const float4 *norm = reinterpret_cast<const float4 *>(a.norm);
    if constexpr (M == Src::Embed) {
        // The token, its row flag and position (scalar loads); the row
        // itself is requested by embed_issue, after the first unit's weights.
        rv.tok = load_uniform(a.tokens + token);
        rv.audio = load_uniform(a.row_flags + token);
        rv.pos = load_uniform(a.pos + token);
    }
    const float4 *row = reinterpret_cast<const float4 *>(a.x + (size_t)token * a.k);
#pragma unroll
    for (int p = 0; p < 3; ++p) {
        if (p * 256 >= (int)k8) break;  // uniform: no thread has values in this stretch
        const uint32_t e8 = tid + p * 256 < k8 ? tid + p * 256 : k8 - 1;
        if constexpr (M != Src::Embed) {
            const float4 lo = row[e8 * 2], hi = row[e8 * 2 + 1];
            rv.v[p][0] = lo.x; rv.v[p][1] = lo.y; rv.v[p][2] = lo.z; rv.v[p][3] = lo.w;
            rv.v[p][4] = hi.x; rv.v[p][5] = hi.y; rv.v[p][6] = hi.z; rv.v[p][7] = hi.w;
        }
        if constexpr (M == Src::RmsNorm || M == Src::Embed) {
            const float4 wl = norm[e8 * 2], wh = norm[e8 * 2 + 1];
            rv.w[p][0] = wl.x; rv.w[p][1] = wl.y; rv.w[p][2] = wl.z; rv.w[p][3] = wl.w;
            rv.w[p][4] = wh.x; rv.w[p][5] = wh.y; rv.w[p][6] = wh.z; rv.w[p][7] = wh.w;
        }
    }
}

// Embed's second phase, after the first unit's weights are requested: the
// token's embedding row (or its audio row) and, in workgroup 0, its RoPE
// row.
template <Src M>
__device__ __forceinline__ void block_late(const GemvQ4Args &a, uint32_t token, RowValues &rv, float &rope) {
    const int tid = threadIdx.x;
    const uint32_t k8 = a.k / 8;
    const uint32_t e8 = (uint32_t)tid < k8 ? tid : k8 - 1;  // one stretch (K <= 2048)
    if constexpr (M == Src::Embed) {
        if (rv.audio) {
            const float4 *row = reinterpret_cast<const float4 *>(a.rows + (size_t)token * a.k);
            const float4 lo = row[e8 * 2], hi = row[e8 * 2 + 1];
            rv.v[0][0] = lo.x; rv.v[0][1] = lo.y; rv.v[0][2] = lo.z; rv.v[0][3] = lo.w;
            rv.v[0][4] = hi.x; rv.v[0][5] = hi.y; rv.v[0][6] = hi.z; rv.v[0][7] = hi.w;
        } else {
            embed_fetch(a, rv.tok, e8, rv.v[0]);
        }
        if (blockIdx.x == 0 && tid < (int)(2 * a.rope_half)) {
            const uint32_t p = rv.pos;
            rope = tid < (int)a.rope_half ? a.rope_cos[(size_t)p * a.rope_half + tid]
                                          : a.rope_sin[(size_t)p * a.rope_half + tid - a.rope_half];
        }
    }
}

template <Src M>
__device__ __forceinline__ void block_encode(const GemvQ4Args &a, const RowValues &rv, ActLds &lds, float rope) {
    const int tid = threadIdx.x;
    const uint32_t k8 = a.k / 8;
    float v[3][8];
#pragma unroll
    for (int p = 0; p < 3; ++p) {
        const bool in = p * 256 < (int)k8 && tid + p * 256 < k8;
#pragma unroll
        for (int i = 0; i < 8; ++i) v[p][i] = in ? rv.v[p][i] : 0.0f;
    }
    if constexpr (M == Src::Embed) {
        // Workgroup 0 of the token stores its row (the residual stream the
        // later projections add to) and its RoPE table row.
        if (blockIdx.x == 0) {
            const uint32_t token = blockIdx.y;
#pragma unroll
            for (int p = 0; p < 3; ++p) {
                if (p * 256 >= (int)k8 || tid + p * 256 >= (int)k8) break;
                float4 *dst = reinterpret_cast<float4 *>(a.hidden_out + (size_t)token * a.k + 8 * (tid + p * 256));
                dst[0] = make_float4(v[p][0], v[p][1], v[p][2], v[p][3]);
                dst[1] = make_float4(v[p][4], v[p][5], v[p][6], v[p][7]);
            }
            if (tid < (int)(2 * a.rope_half)) a.rope_now[(size_t)token * 2 * a.rope_half + tid] = rope;
        }
    }
    if constexpr (M == Src::RmsNorm || M == Src::Embed) {
        // math.zig:120-130: x * (1 / sqrt(mean(x^2) + eps)) * w, the sum of
        // squares reduced over the block (threads, then the four waves in
        // order).
        float w[3][8];
#pragma unroll
        for (int p = 0; p < 3; ++p)
#pragma unroll
            for (int i = 0; i < 8; ++i) w[p][i] = p * 256 < (int)k8 ? rv.w[p][i] : 0.0f;
        float ss = 0.0f;
#pragma unroll
        for (int p = 0; p < 3; ++p)
#pragma unroll
            for (int i = 0; i < 8; ++i) ss = __fadd_rn(ss, __fmul_rn(v[p][i], v[p][i]));
        ss = dev::wave_sum(ss);
        if ((tid & 63) == 0) lds.partial[tid >> 6] = ss;
        __syncthreads();
        ss = ((lds.partial[0] + lds.partial[1]) + lds.partial[2]) + lds.partial[3];
        const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)a.k), a.eps)));
#pragma unroll
        for (int p = 0; p < 3; ++p)
#pragma unroll
            for (int i = 0; i < 8; ++i) v[p][i] = __fmul_rn(__fmul_rn(v[p][i], inv), w[p][i]);
    }
#pragma unroll
    for (int p = 0; p < 3; ++p) {
        const uint32_t e8 = tid + p * 256;
        if (p * 256 >= (int)k8) break;  // uniform: no thread has values in this stretch
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[p][i]));
        amax = fmaxf(amax, dev::xor_lane<1>(amax));
        amax = fmaxf(amax, dev::xor_lane<2>(amax));
        const int e = dev::chunk_exponent(amax);
        uint32_t planes[6];
        dev::encode_digits8(v[p], e, planes);
        if (e8 < k8) {
            const uint32_t chunk = e8 >> 2;
            const uint32_t q = e8 & 3u;
#pragma unroll
            for (int j = 0; j < 6; ++j) lds.words[chunk * 24 + j * 4 + q] = planes[j];
            if (q == 0) lds.mult[chunk] = __builtin_ldexpf(1.0f, e - 22);
        }
    }
    __syncthreads();
}

// This lane's activation operands for slices c = li + s * L: from the
// prepared planes in global memory, or from the block's LDS encoding.
template <int S, int L, Src M>
__device__ __forceinline__ void lane_activations(const GemvQ4Args &a, int li, uint32_t token,
                                                 uint32_t (&D)[S][24], float (&m)[S], const ActLds &lds) {
    const uint32_t T = a.t;
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const uint32_t c = li + s * L;
        const uint4 *src = M == Src::Digits
                               ? reinterpret_cast<const uint4 *>(a.words + ((size_t)token * T + c) * 24)
                               : reinterpret_cast<const uint4 *>(&lds.words[c * 24]);
#pragma unroll
        for (int j = 0; j < 6; ++j) {
            const uint4 w = src[j];
            D[s][j * 4 + 0] = w.x;
            D[s][j * 4 + 1] = w.y;
            D[s][j * 4 + 2] = w.z;
            D[s][j * 4 + 3] = w.w;
        }
        m[s] = M == Src::Digits ? a.mult[(size_t)token * T + c] : lds.mult[c];
    }
}

// The wavefront takes every nwaves-th unit (U row groups of RG = 64/L rows
// each). Lane l works on row l / L of each row group and on slices
// (l % L) + s * L, s < S, of that row.
template <int S, int L, int U, Src M>
__global__ __launch_bounds__(256) void gemv_q4_kernel(const GemvQ4Args a) {
    constexpr int RG = 64 / L;
    constexpr int log_l = Log2<L>::value;
    constexpr int log_u = Log2<U>::value;
    const int lane = threadIdx.x & 63;
    const int rr = lane >> log_l;
    const int li = lane & (L - 1);
    // Wave-uniform (scalar) indices: the unit loop and the full/tail choice
    // branch on scalars instead of masking lanes.
    const uint32_t wave = __builtin_amdgcn_readfirstlane(blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6));
    const uint32_t nwaves = gridDim.x * (blockDim.x >> 6);
    const uint32_t token = blockIdx.y;
    const uint32_t gpr = a.k >> 6;
    // The launcher picks this kernel only when the data plane is below 4 GiB
    // and units * waves fits 32 bits, so 32-bit arithmetic suffices.
    const uint32_t row_bytes = a.k >> 1;
    const uint32_t units = (a.row_groups + U - 1) / U;
    const uint32_t full_units = a.n / (U * RG);
    // Grid-stride units: wave w takes units w, w + nwaves, ..., so at any
    // moment the waves stream one compact window of the matrix.
    const uint32_t count = full_units > wave ? (full_units - wave + nwaves - 1) / nwaves : 0;
    float *out = a.out + (size_t)token * (a.pairs ? a.n / 2 : a.n);
    const float *residual = a.residual ? a.residual + (size_t)token * a.n : nullptr;

    // Unmasked loads of a unit whose rows all exist.
    auto load = [&](Slice (&dst)[U][S], uint32_t unit) {
        const uint32_t row0 = unit * (U * RG) + rr;
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const uint32_t row = row0 + u * RG;
                const uint32_t c = li + s * L;
                dst[u][s].codes = load_stream16(a.data + (row * row_bytes + c * 16));
                dst[u][s].scale = load_scale(a.scales, row * gpr + (c >> 1));
            }
    };
    // The last, partial unit: rows past the end contribute nothing.
    auto load_tail = [&](Slice (&dst)[U][S], uint32_t unit) {
        const uint32_t row0 = unit * (U * RG) + rr;
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const uint32_t row = row0 + u * RG;
                const uint32_t c = li + s * L;
                if (row < a.n) {
                    dst[u][s].codes = load_stream16(a.data + (row * row_bytes + c * 16));
                    dst[u][s].scale = load_scale(a.scales, row * gpr + (c >> 1));
                } else {
                    dst[u][s].codes = make_uint4(0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u);
                    dst[u][s].scale = 0;
                }
            }
    };

    // The residual of the row this lane writes for a unit, fetched with the
    // unit's weights so the epilogue does not wait on another load.
    auto load_res = [&](uint32_t unit) -> float {
        const uint32_t row = (unit * U + (li >> (log_l - log_u))) * RG + rr;
        return residual && row < a.n ? residual[row] : 0.0f;
    };

    Slice A[U][S], B[U][S];
    float resA = 0.0f, resB = 0.0f;
    // Issue order: the row's values, then the first unit's weights, so that
    // their latency covers the encoding. The weight loads are unconditional
    // (a wave without full units loads a clamped unit it never uses): a
    // branch around them would make the wait for the row's values wait for
    // them as well.
    RowValues rv;
    if constexpr (M != Src::Digits) block_fetch<M>(a, token, rv);
    {
        const uint32_t first = count ? wave : (full_units ? full_units - 1 : 0);
        const uint32_t row0 = first * (U * RG) + rr;
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const uint32_t row = row0 + u * RG < a.n ? row0 + u * RG : a.n - 1;
                const uint32_t c = li + s * L;
                A[u][s].codes = load_stream16(a.data + (row * row_bytes + c * 16));
                A[u][s].scale = load_scale(a.scales, row * gpr + (c >> 1));
            }
    }

    float rope = 0.0f;
    if constexpr (M == Src::Embed) block_late<M>(a, token, rv, rope);
    __shared__ __attribute__((aligned(16))) ActLds lds;
    if constexpr (M != Src::Digits) block_encode<M>(a, rv, lds, rope);
    uint32_t D[S][24];
    float m[S];
    lane_activations<S, L, M>(a, li, token, D, m, lds);
    if (count) resA = load_res(wave);

    // Argmax partials: this lane's best (value, row) of the rows it writes.
    const bool track = a.arg_value != nullptr;
    float best_v = -FLT_MAX;
    uint32_t best_i = 0xffffffffu;
    auto process = [&](const Slice (&src)[U][S], float res, uint32_t unit) {
        float acc[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const float part = (float)q4_slice_dot(src[u][s].codes, D[s]) *
                                   (dev::f16_bits_to_f32(src[u][s].scale) * m[s]);
                acc[u] = s == 0 ? part : acc[u] + part;
            }
        }
        const float total = reduce_rows<U, L>(acc, lane);
        const bool writer = (li & ((L >> log_u) - 1)) == 0;
        const uint32_t row = (unit * U + (li >> (log_l - log_u))) * RG + rr;
        if (a.pairs) {
            // Row + 1 sits in the next row of the row group (RG > 1), else
            // in the next of the unit's U row groups.
            const float partner = __shfl_down(total, RG > 1 ? L : (L >> log_u), kWave);
            if (writer && (row & 1u) == 0 && row < a.n) out[row >> 1] = silu_mul(total, partner);
        } else if (writer && row < a.n) {
            const float y = res + total;
            out[row] = y;
            // A NaN first output is argmaxLogits' answer (no value compares
            // greater than it): row 0 then wins outright.
            if (track) arg_better(best_v, best_i, row == 0 && y != y ? INFINITY : y, row);
        }
    };

    // Full units, software pipelined: the loads of the next unit are in
    // flight while the current one is multiplied. The prefetch index is
    // clamped rather than branched on, so the body is straight-line code and
    // the wait before each multiply covers only that unit's loads.
    uint32_t i = 0;
    for (; i + 1 < count; i += 2) {
        const uint32_t ua = wave + i * nwaves, ub = ua + nwaves;
        load(B, ub);
        resB = load_res(ub);
        process(A, resA, ua);
        const uint32_t un = i + 2 < count ? ub + nwaves : ub;
        load(A, un);
        resA = load_res(un);
        process(B, resB, ub);
    }
    if (i < count) process(A, resA, wave + i * nwaves);
    // The partial unit (rows past the end contribute nothing), taken by the
    // wave whose stride reaches it.
    if (full_units < units && full_units % nwaves == wave) {
        load_tail(B, full_units);
        process(B, load_res(full_units), full_units);
    }
    if (track) {
        // The workgroup's best: the wavefront's lanes, then its four waves.
#pragma unroll
        for (int mask = 32; mask >= 1; mask >>= 1)
            arg_better(best_v, best_i, __shfl_xor(best_v, mask, kWave), __shfl_xor(best_i, mask, kWave));
        __shared__ float arg_v[4];
        __shared__ uint32_t arg_i[4];
        if (lane == 0) {
            arg_v[threadIdx.x >> 6] = best_v;
            arg_i[threadIdx.x >> 6] = best_i;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
#pragma unroll
            for (int w = 1; w < 4; ++w) arg_better(best_v, best_i, arg_v[w], arg_i[w]);
            a.arg_value[(size_t)token * gridDim.x + blockIdx.x] = best_v;
            a.arg_index[(size_t)token * gridDim.x + blockIdx.x] = best_i;
        }
    }
}

// Any K (a multiple of 64): one wavefront per row, lanes stride over the
// row's 16-byte slices and read the digit planes from memory.
__global__ __launch_bounds__(256) void gemv_q4_generic_kernel(const GemvQ4Args a) {
    const int lane = threadIdx.x & 63;
    const uint32_t wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const uint32_t nwaves = (gridDim.x * blockDim.x) >> 6;
    const uint32_t token = blockIdx.y;
    const uint32_t T = a.t;
    const uint32_t gpr = a.k >> 6;
    const size_t row_bytes = a.k >> 1;
    float *out = a.out + (size_t)token * (a.pairs ? a.n / 2 : a.n);
    const float *residual = a.residual ? a.residual + (size_t)token * a.n : nullptr;
    auto row_dot = [&](uint32_t row) {
        float acc = 0.0f;
        for (uint32_t c = lane; c < T; c += 64) {
            const uint4 code = reinterpret_cast<const uint4 *>(a.data + row * row_bytes)[c];
            uint32_t d[24];
            const uint4 *src = reinterpret_cast<const uint4 *>(a.words + ((size_t)token * T + c) * 24);
#pragma unroll
            for (int j = 0; j < 6; ++j) {
                const uint4 w = src[j];
                d[j * 4 + 0] = w.x; d[j * 4 + 1] = w.y; d[j * 4 + 2] = w.z; d[j * 4 + 3] = w.w;
            }
            const float mult = a.mult[(size_t)token * T + c];
            acc += (float)q4_slice_dot(code, d) * (dev::f16_bits_to_f32(a.scales[(size_t)row * gpr + (c >> 1)]) * mult);
        }
        return dev::wave_sum(acc);
    };
    if (a.pairs) {
        // Rows 2 j (gate) and 2 j + 1 (up) in one wavefront: siluMul.
        for (uint32_t j = wave; 2 * j + 1 < a.n; j += nwaves) {
            const float g = row_dot(2 * j), u = row_dot(2 * j + 1);
            if (lane == 0) out[j] = silu_mul(g, u);
        }
        return;
    }
    for (uint32_t row = wave; row < a.n; row += nwaves) {
        const float acc = row_dot(row);
        if (lane == 0) out[row] = (residual ? residual[row] : 0.0f) + acc;
    }
}

// ---------------------------------------------------------------------------
// q8: slices of 16 codes; the lane's activations (16 f32 per slot) stay in
// registers. Codes convert exactly to f32 and the bias is subtracted before
// the multiply, so each product is the reference's decoded weight times x up
// to the group scale, applied once per slice.
// ---------------------------------------------------------------------------
struct GemvQ8Args {
    const float *x;         // tokens x K
    const uint16_t *scales; // N * K/64
    const uint8_t *data;    // N * K
    float *out;
    const float *residual;
    uint32_t n, k, t, row_groups;  // t = K/16 slices per row
};

__device__ __forceinline__ float q8_slice_dot(const uint4 codes, const float (&x)[16]) {
    float acc = 0.0f;
    const uint32_t w[4] = {codes.x, codes.y, codes.z, codes.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const float c = (float)((w[i] >> (8 * b)) & 0xffu) - 128.0f;
            acc = fmaf(c, x[i * 4 + b], acc);
        }
    }
    return acc;
}

template <int S, int L, int U>
__global__ __launch_bounds__(256) void gemv_q8_kernel(const GemvQ8Args a) {
    constexpr int RG = 64 / L;
    constexpr int log_l = Log2<L>::value;
    constexpr int log_u = Log2<U>::value;
    const int lane = threadIdx.x & 63;
    const int rr = lane >> log_l;
    const int li = lane & (L - 1);
    const uint32_t wave = __builtin_amdgcn_readfirstlane(blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6));
    const uint32_t nwaves = gridDim.x * (blockDim.x >> 6);
    const uint32_t token = blockIdx.y;
    const uint32_t gpr = a.k >> 6;
    float X[S][16];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const uint32_t c = li + s * L;
        const float4 *src = reinterpret_cast<const float4 *>(a.x + (size_t)token * a.k + c * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = src[i];
            X[s][i * 4 + 0] = v.x; X[s][i * 4 + 1] = v.y; X[s][i * 4 + 2] = v.z; X[s][i * 4 + 3] = v.w;
        }
    }
    const uint32_t units = (a.row_groups + U - 1) / U;
    const uint32_t u0 = wave * units / nwaves;
    const uint32_t u1 = (wave + 1) * units / nwaves;
    float *out = a.out + (size_t)token * a.n;
    const float *residual = a.residual ? a.residual + (size_t)token * a.n : nullptr;
    for (uint32_t unit = u0; unit < u1; ++unit) {
        Slice sl[U][S];
        const uint32_t row0 = unit * (U * RG) + rr;
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const uint32_t row = row0 + u * RG;
                const uint32_t c = li + s * L;
                if (row < a.n) {
                    sl[u][s].codes = load_stream16(a.data + (row * a.k + c * 16));
                    sl[u][s].scale = load_scale(a.scales, row * gpr + (c >> 2));
                } else {
                    sl[u][s].codes = make_uint4(0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u);
                    sl[u][s].scale = 0;
                }
            }
        float acc[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const float part = q8_slice_dot(sl[u][s].codes, X[s]) * dev::f16_bits_to_f32(sl[u][s].scale);
                acc[u] = s == 0 ? part : acc[u] + part;
            }
        }
        const float total = reduce_rows<U, L>(acc, lane);
        if ((li & ((L >> log_u) - 1)) == 0) {
            const uint32_t row = (unit * U + (li >> (log_l - log_u))) * RG + rr;
            if (row < a.n) out[row] = (residual ? residual[row] : 0.0f) + total;
        }
    }
}

__global__ __launch_bounds__(256) void gemv_q8_generic_kernel(const GemvQ8Args a) {
    const int lane = threadIdx.x & 63;
    const uint32_t wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const uint32_t nwaves = (gridDim.x * blockDim.x) >> 6;
    const uint32_t token = blockIdx.y;
    const uint32_t gpr = a.k >> 6;
    float *out = a.out + (size_t)token * a.n;
    const float *residual = a.residual ? a.residual + (size_t)token * a.n : nullptr;
    for (uint32_t row = wave; row < a.n; row += nwaves) {
        float acc = 0.0f;
        for (uint32_t c = lane; c < a.t; c += 64) {
            const uint4 code = reinterpret_cast<const uint4 *>(a.data + (size_t)row * a.k)[c];
            float x[16];
            const float4 *src = reinterpret_cast<const float4 *>(a.x + (size_t)token * a.k + c * 16);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 v = src[i];
                x[i * 4 + 0] = v.x; x[i * 4 + 1] = v.y; x[i * 4 + 2] = v.z; x[i * 4 + 3] = v.w;
            }
            acc += q8_slice_dot(code, x) * dev::f16_bits_to_f32(a.scales[(size_t)row * gpr + (c >> 2)]);
        }
        acc = dev::wave_sum(acc);
        if (lane == 0) out[row] = (residual ? residual[row] : 0.0f) + acc;
    }
}

// ---------------------------------------------------------------------------
// Byte-plane GEMV for q5 and q8 (quant.zig:253-269 and :270-288 planes).
//
// A lane takes a 32-column half group ("slice") of its row:
//   q5  two 8-byte loads of nibbles (a group is 40 bytes: 32 bytes of low
//       nibbles, even column in the low nibble, then 8 bytes of fifth bits,
//       bit j % 8 of byte j / 8 for column j; so a slice is only 8-byte
//       aligned) and the slice's 4 bytes of fifth bits;
//   q8  two 16-byte loads of 32 codes.
//
// Arithmetic. The codes are turned into bytes in one fixed column order:
// within each 8-column block, columns {0,2,4,6} then {1,3,5,7}.
//   q5  a nibble mask splits the packed bytes that way; the fifth bits of
//       those four columns are bits 0,2,4,6 of one byte, moved to bit 4 of
//       bytes 0..3 by one multiply ((b & 0x55) * 0x00410410 has them at bits
//       4, 12, 20, 28 and no carry reaches those bits): u = nibble |
//       fifth << 4 in [0, 31];
//   q8  v_perm_b32 picks the even and the odd bytes of the block's two code
//       words, and XOR 0x80 makes each byte the signed code u - 128.
// The activations of a 32-column chunk are written as x_int = rint(x *
// 2^(22-e)) (2^e bounds the chunk's |x|) in three signed base-256 digit
// planes d0 + 256 d1 + 65536 d2, stored in the same column order, so that
// v_dot4_i32_i8 multiplies matching columns. With S_j the chunk's sum of plane
// j's digits,
//     q5: sum (u - 16) x_int = sum_j 256^j (sum u d_j - 16 S_j),
//     q8: sum (u - 128) x_int = sum_j 256^j sum (u - 128) d_j,
// each plane's term exact in int32 (below 2^19), combined in f32 and scaled
// by the group's f16 scale times 2^(e-22).
//
// The activations are f32 values each workgroup encodes into LDS once (as
// they are, or after RMSNorm, kernels.zig:274-300); the output is the row
// products plus an optional residual, or siluMul of gate / up row pairs
// (kernels.zig:233-239), as in the q4 kernel.
// ---------------------------------------------------------------------------
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

enum class Fmt8 : int { Q5 = 0, Q8 = 1 };

template <Fmt8 F>
struct Slice8;
template <>
struct Slice8<Fmt8::Q5> {
    u32x2 lo0, lo1;  // nibbles of columns 0..15 and 16..31
    uint32_t hi;     // fifth bits of columns 0..31 (byte q: columns 8q..8q+7)
    uint16_t scale;
};
template <>
struct Slice8<Fmt8::Q8> {
    u32x4 a, b;      // codes of columns 0..15 and 16..31
    uint16_t scale;
};

struct Act8Lds {
    uint32_t words[kMaxChunks * 24];  // chunk c: plane j dword m at 24c + 8j + m
    int sums[kMaxChunks * 4];         // chunk c: S_j at 4c + j
    float mult[kMaxChunks];
    float partial[4];                 // RMSNorm: the waves' sums of squares
};

struct GemvB8Args {
    const float *x;         // tokens x K
    const float *norm;      // RmsNorm: K weights
    float eps;
    const uint16_t *scales; // N * K/64
    const uint8_t *data;    // q5: N * K/64 * 40, q8: N * K
    float *out;             // tokens x N, or tokens x N/2 with pairs
    const float *residual;  // optional, tokens x N (may alias out); not with pairs
    uint32_t n, k, t, row_groups;  // t = K/32 slices per row
    uint32_t pairs;         // rows 2j, 2j+1 are gate_j, up_j: write silu(gate_j) * up_j
};

template <Fmt8 F>
__device__ __forceinline__ uint32_t b8_row_bytes(uint32_t gpr) {
    return F == Fmt8::Q5 ? gpr * 40u : gpr * 64u;
}

// The row's values (and RMSNorm weights) this thread encodes: thread t takes
// values 8t .. 8t+7 of each 2048-value stretch (threads past the row's end
// load its last 8 values and drop them when encoding). Fetched before the
// first unit's weights are requested, so the wait for them leaves the weight
// loads in flight.
template <Src M>
__device__ __forceinline__ void fetch_row(const float *x, const float *norm, uint32_t k, RowValues &rv) {
    const int tid = threadIdx.x;
    const uint32_t k8 = k / 8;
    const float4 *row = reinterpret_cast<const float4 *>(x);
    const float4 *w = reinterpret_cast<const float4 *>(norm);
#pragma unroll
    for (int p = 0; p < 3; ++p) {
        if (p * 256 >= (int)k8) break;  // uniform
        const uint32_t e8 = tid + p * 256 < k8 ? tid + p * 256 : k8 - 1;
        const float4 lo = row[e8 * 2], hi = row[e8 * 2 + 1];
        rv.v[p][0] = lo.x; rv.v[p][1] = lo.y; rv.v[p][2] = lo.z; rv.v[p][3] = lo.w;
        rv.v[p][4] = hi.x; rv.v[p][5] = hi.y; rv.v[p][6] = hi.z; rv.v[p][7] = hi.w;
        if constexpr (M == Src::RmsNorm) {
            const float4 wl = w[e8 * 2], wh = w[e8 * 2 + 1];
            rv.w[p][0] = wl.x; rv.w[p][1] = wl.y; rv.w[p][2] = wl.z; rv.w[p][3] = wl.w;
            rv.w[p][4] = wh.x; rv.w[p][5] = wh.y; rv.w[p][6] = wh.z; rv.w[p][7] = wh.w;
        }
    }
}

// Encodes the fetched row into LDS as byte digit planes (block-wide; four
// consecutive threads per 32-value chunk), after RMSNorm (math.zig:120-130:
// x * (1 / sqrt(mean(x^2) + eps)) * w, the sum of squares reduced over the
// block in a fixed order) in that form.
template <Src M>
__device__ __forceinline__ void block_encode8(const RowValues &rv, uint32_t k, float eps, Act8Lds &lds) {
    const int tid = threadIdx.x;
    const uint32_t k8 = k / 8;
    float v[3][8];
#pragma unroll
    for (int p = 0; p < 3; ++p) {
        const bool in = p * 256 < (int)k8 && tid + p * 256 < k8;
#pragma unroll
        for (int i = 0; i < 8; ++i) v[p][i] = in ? rv.v[p][i] : 0.0f;
    }
    if constexpr (M == Src::RmsNorm) {
        float ss = 0.0f;
#pragma unroll
        for (int p = 0; p < 3; ++p)
#pragma unroll
            for (int i = 0; i < 8; ++i) ss = __fadd_rn(ss, __fmul_rn(v[p][i], v[p][i]));
        ss = dev::wave_sum(ss);
        if ((tid & 63) == 0) lds.partial[tid >> 6] = ss;
        __syncthreads();
        ss = ((lds.partial[0] + lds.partial[1]) + lds.partial[2]) + lds.partial[3];
        const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)k), eps)));
#pragma unroll
        for (int p = 0; p < 3; ++p)
#pragma unroll
            for (int i = 0; i < 8; ++i)
                v[p][i] = p * 256 < (int)k8 ? __fmul_rn(__fmul_rn(v[p][i], inv), rv.w[p][i]) : 0.0f;
    }
#pragma unroll
    for (int p = 0; p < 3; ++p) {
        if (p * 256 >= (int)k8) break;  // uniform
        const uint32_t e8 = tid + p * 256;
        const bool in = e8 < k8;
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[p][i]));
        amax = fmaxf(amax, dev::xor_lane<1>(amax));
        amax = fmaxf(amax, dev::xor_lane<2>(amax));
        const int e = dev::chunk_exponent(amax);
        const float up = __builtin_ldexpf(1.0f, 22 - e);
        // Bytes 0..2 of u[i] are the signed digits d0, d1, d2 of x_int
        // (adding 0x808080 makes each digit d + 128 with no carries).
        uint32_t u[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) u[i] = (uint32_t)((int)__builtin_rintf(v[p][i] * up) + 0x808080) ^ 0x808080u;
        uint32_t planes[6];
        int sums[3];
#pragma unroll
        for (int j = 0; j < 3; ++j) {
#pragma unroll
            for (int par = 0; par < 2; ++par) {
                uint32_t w = 0;
#pragma unroll
                for (int b = 0; b < 4; ++b) w |= ((u[2 * b + par] >> (8 * j)) & 0xffu) << (8 * b);
                planes[2 * j + par] = w;
            }
            int sj = __builtin_amdgcn_sdot4((int)planes[2 * j], 0x01010101, 0, false);
            sj = __builtin_amdgcn_sdot4((int)planes[2 * j + 1], 0x01010101, sj, false);
            sj += __builtin_bit_cast(int, dev::xor_lane<1>(__builtin_bit_cast(float, sj)));
            sj += __builtin_bit_cast(int, dev::xor_lane<2>(__builtin_bit_cast(float, sj)));
            sums[j] = sj;
        }
        if (in) {
            const uint32_t chunk = e8 >> 2;
            const uint32_t q = e8 & 3u;
#pragma unroll
            for (int j = 0; j < 3; ++j) {
                lds.words[chunk * 24 + j * 8 + 2 * q] = planes[2 * j];
                lds.words[chunk * 24 + j * 8 + 2 * q + 1] = planes[2 * j + 1];
            }
            if (q == 0) {
                lds.mult[chunk] = __builtin_ldexpf(1.0f, e - 22);
#pragma unroll
                for (int j = 0; j < 3; ++j) lds.sums[chunk * 4 + j] = sums[j];
            }
        }
    }
    __syncthreads();
}

// The activation operands of chunk c from LDS: digit planes, the bias term
// that starts each plane's dot chain (q5: -16 times the plane's digit sum;
// q8: none), and the chunk multiplier.
struct Act8 {
    uint32_t d[24];
    int bias[3];
    float mult;
};

template <Fmt8 F>
__device__ __forceinline__ void load_act8(const Act8Lds &lds, uint32_t c, Act8 &x) {
    const uint4 *src = reinterpret_cast<const uint4 *>(&lds.words[c * 24]);
#pragma unroll
    for (int j = 0; j < 6; ++j) {
        const uint4 w = src[j];
        x.d[j * 4 + 0] = w.x;
        x.d[j * 4 + 1] = w.y;
        x.d[j * 4 + 2] = w.z;
        x.d[j * 4 + 3] = w.w;
    }
    if constexpr (F == Fmt8::Q5) {
        const int4 sv = *reinterpret_cast<const int4 *>(&lds.sums[c * 4]);
        x.bias[0] = -16 * sv.x;
        x.bias[1] = -16 * sv.y;
        x.bias[2] = -16 * sv.z;
    } else {
        x.bias[0] = x.bias[1] = x.bias[2] = 0;
    }
    x.mult = lds.mult[c];
}

// sum (u - bias) x_int of one slice, in f32 (the integer plane terms exact).
__device__ __forceinline__ float b8_slice_dot(const Slice8<Fmt8::Q5> &sl, const Act8 &x) {
    const uint32_t w[4] = {sl.lo0.x, sl.lo0.y, sl.lo1.x, sl.lo1.y};
    // Fifth bits of the even and of the odd columns, each byte's four at bits
    // 0, 2, 4, 6 (so one bit-field extract per byte below).
    const uint32_t fifths[2] = {sl.hi & 0x55555555u, (sl.hi >> 1) & 0x55555555u};
    int p0 = x.bias[0], p1 = x.bias[1], p2 = x.bias[2];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
        for (int par = 0; par < 2; ++par) {
            const uint32_t nib = (par ? w[q] >> 4 : w[q]) & 0x0f0f0f0fu;
            const uint32_t bits = __builtin_amdgcn_ubfe(fifths[par], 8 * q, 8);
            const int um = (int)(((bits * 0x00410410u) & 0x10101010u) | nib);
            const int m = 2 * q + par;
            p0 = __builtin_amdgcn_sdot4(um, (int)x.d[m], p0, false);
            p1 = __builtin_amdgcn_sdot4(um, (int)x.d[8 + m], p1, false);
            p2 = __builtin_amdgcn_sdot4(um, (int)x.d[16 + m], p2, false);
        }
    }
    return ((float)p2 * 65536.0f + (float)p1 * 256.0f) + (float)p0;
}

__device__ __forceinline__ float b8_slice_dot(const Slice8<Fmt8::Q8> &sl, const Act8 &x) {
    const uint32_t w[8] = {sl.a.x, sl.a.y, sl.a.z, sl.a.w, sl.b.x, sl.b.y, sl.b.z, sl.b.w};
    int p0 = 0, p1 = 0, p2 = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        // Bytes of columns {0,2,4,6} and {1,3,5,7} of block q, as u - 128.
        const int even = (int)(__builtin_amdgcn_perm(w[2 * q + 1], w[2 * q], 0x06040200u) ^ 0x80808080u);
        const int odd = (int)(__builtin_amdgcn_perm(w[2 * q + 1], w[2 * q], 0x07050301u) ^ 0x80808080u);
        const int m = 2 * q;
        p0 = __builtin_amdgcn_sdot4(even, (int)x.d[m], p0, false);
        p1 = __builtin_amdgcn_sdot4(even, (int)x.d[8 + m], p1, false);
        p2 = __builtin_amdgcn_sdot4(even, (int)x.d[16 + m], p2, false);
        p0 = __builtin_amdgcn_sdot4(odd, (int)x.d[m + 1], p0, false);
        p1 = __builtin_amdgcn_sdot4(odd, (int)x.d[8 + m + 1], p1, false);
        p2 = __builtin_amdgcn_sdot4(odd, (int)x.d[16 + m + 1], p2, false);
    }
    return ((float)p2 * 65536.0f + (float)p1 * 256.0f) + (float)p0;
}

template <Fmt8 F>
__device__ __forceinline__ Slice8<F> load_slice8(const GemvB8Args &a, uint32_t row, uint32_t c, uint32_t row_bytes,
                                                 uint32_t gpr) {
    Slice8<F> sl;
    if constexpr (F == Fmt8::Q5) {
        const uint8_t *base = a.data + (row * row_bytes + (c >> 1) * 40u);
        sl.lo0 = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(base + (c & 1u) * 16u));
        sl.lo1 = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(base + (c & 1u) * 16u + 8u));
        sl.hi = __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(base + 32u + (c & 1u) * 4u));
    } else {
        const uint8_t *base = a.data + (row * row_bytes + c * 32u);
        sl.a = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(base));
        sl.b = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(base + 16u));
    }
    sl.scale = load_scale(a.scales, row * gpr + (c >> 1));
    return sl;
}

// Lane mapping and unit walk as the q4 kernel (RG = 64/L rows per row group,
// S slices per lane, U row groups per unit, grid-stride units, the next
// unit's loads issued before the current one is multiplied; the row's
// values are fetched before the first weights).
template <Fmt8 F, int S, int L, int U, Src M>
__global__ __launch_bounds__(256) void gemv_b8_kernel(const GemvB8Args a) {
    constexpr int RG = 64 / L;
    constexpr int log_l = Log2<L>::value;
    constexpr int log_u = Log2<U>::value;
    const int lane = threadIdx.x & 63;
    const int rr = lane >> log_l;
    const int li = lane & (L - 1);
    const uint32_t wave = __builtin_amdgcn_readfirstlane(blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6));
    const uint32_t nwaves = gridDim.x * (blockDim.x >> 6);
    const uint32_t token = blockIdx.y;
    const uint32_t gpr = a.k >> 6;
    const uint32_t row_bytes = b8_row_bytes<F>(gpr);
    const uint32_t units = (a.row_groups + U - 1) / U;
    const uint32_t full_units = a.n / (U * RG);
    const uint32_t count = full_units > wave ? (full_units - wave + nwaves - 1) / nwaves : 0;
    float *out = a.out + (size_t)token * (a.pairs ? a.n / 2 : a.n);
    const float *residual = a.residual ? a.residual + (size_t)token * a.n : nullptr;

    // Rows past the end (only in the last, partial unit) load the last row
    // and are dropped at the store.
    auto load = [&](Slice8<F> (&dst)[U][S], uint32_t unit) __attribute__((always_inline)) {
        const uint32_t row0 = unit * (U * RG) + rr;
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const uint32_t row = row0 + u * RG < a.n ? row0 + u * RG : a.n - 1;
                dst[u][s] = load_slice8<F>(a, row, li + s * L, row_bytes, gpr);
            }
    };
    auto load_res = [&](uint32_t unit) -> float {
        const uint32_t row = (unit * U + (li >> (log_l - log_u))) * RG + rr;
        return residual && row < a.n ? residual[row] : 0.0f;
    };

    Slice8<F> A[U][S], B[U][S];
    RowValues rv;
    fetch_row<M>(a.x + (size_t)token * a.k, a.norm, a.k, rv);
    load(A, count ? wave : (full_units ? full_units - 1 : 0));
    __shared__ __attribute__((aligned(16))) Act8Lds lds;
    block_encode8<M>(rv, a.k, a.eps, lds);
    Act8 X[S];
#pragma unroll
    for (int s = 0; s < S; ++s) load_act8<F>(lds, li + s * L, X[s]);
    float resA = count ? load_res(wave) : 0.0f, resB = 0.0f;

    auto process = [&](const Slice8<F> (&src)[U][S], float res, uint32_t unit) __attribute__((always_inline)) {
        float acc[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const float part = b8_slice_dot(src[u][s], X[s]) * (dev::f16_bits_to_f32(src[u][s].scale) * X[s].mult);
                acc[u] = s == 0 ? part : acc[u] + part;
            }
        }
        const float total = reduce_rows<U, L>(acc, lane);
        const bool writer = (li & ((L >> log_u) - 1)) == 0;
        const uint32_t row = (unit * U + (li >> (log_l - log_u))) * RG + rr;
        if (a.pairs) {
            // Row + 1 sits in the next row of the row group (RG > 1), else
            // in the next of the unit's U row groups.
            const float partner = __shfl_down(total, RG > 1 ? L : (L >> log_u), kWave);
            if (writer && (row & 1u) == 0 && row < a.n) out[row >> 1] = silu_mul(total, partner);
        } else if (writer && row < a.n) {
            out[row] = res + total;
        }
    };

    uint32_t i = 0;
    for (; i + 1 < count; i += 2) {
        const uint32_t ua = wave + i * nwaves, ub = ua + nwaves;
        load(B, ub);
        resB = load_res(ub);
        process(A, resA, ua);
        const uint32_t un = i + 2 < count ? ub + nwaves : ub;
        load(A, un);
        resA = load_res(un);
        process(B, resB, ub);
    }
    if (i < count) process(A, resA, wave + i * nwaves);
    if (full_units < units && full_units % nwaves == wave) {
        load(B, full_units);
        process(B, load_res(full_units), full_units);
    }
}

// q5 with the unit's bytes loaded whole: a unit's U RG rows are one
// contiguous stretch of the data plane (1280 U S bytes, a whole number of
// 16-byte pieces), which the wavefront loads as consecutive 16-byte pieces
// (clamped to the plane's end) and passes through its own LDS, from which
// each lane reads its slices' 16 nibble bytes and 4 fifth-bit bytes. The
// per-lane form needs four loads per slice (two 8-byte, one 4-byte and the
// scale); this one 1.25 plus the scale. Otherwise as gemv_b8_kernel.
template <int S, int L, int U, Src M>
__global__ __launch_bounds__(256) void gemv_q5_staged_kernel(const GemvB8Args a) {
    constexpr int RG = 64 / L;
    constexpr int log_l = Log2<L>::value;
    constexpr int log_u = Log2<U>::value;
    constexpr uint32_t UB = 1280u * U * S;  // bytes per unit: U RG rows of 20 S L bytes
    constexpr int P = UB / 16, NWQ = (P + 63) / 64;
    const int lane = threadIdx.x & 63;
    const int rr = lane >> log_l;
    const int li = lane & (L - 1);
    const uint32_t wave = __builtin_amdgcn_readfirstlane(blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6));
    const uint32_t nwaves = gridDim.x * (blockDim.x >> 6);
    const uint32_t token = blockIdx.y;
    const uint32_t gpr = a.k >> 6;
    const uint32_t row_bytes = b8_row_bytes<Fmt8::Q5>(gpr);
    const uint32_t units = (a.row_groups + U - 1) / U;
    const uint32_t full_units = a.n / (U * RG);
    const uint32_t count = full_units > wave ? (full_units - wave + nwaves - 1) / nwaves : 0;
    const uint32_t last_piece = a.n * row_bytes - 16;
    float *out = a.out + (size_t)token * (a.pairs ? a.n / 2 : a.n);
    const float *residual = a.residual ? a.residual + (size_t)token * a.n : nullptr;
    __shared__ u32x4 wst[4][P];
    u32x4 *wl = wst[threadIdx.x >> 6];

    struct Unit {
        u32x4 w[NWQ];
        uint16_t scale[U][S];
    };
    // Pieces past the plane's end read its last piece again; rows past the
    // end are dropped at the store.
    auto load = [&](Unit &dst, uint32_t unit) __attribute__((always_inline)) {
        const uint32_t base = unit * UB;
#pragma unroll
        for (int m = 0; m < NWQ; ++m) {
            const uint32_t q = lane + 64 * m < P ? lane + 64 * m : P - 1;
            const uint32_t off = min(base + 16u * q, last_piece);
            dst.w[m] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(a.data + off));
        }
        const uint32_t row0 = unit * (U * RG) + rr;
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const uint32_t row = row0 + u * RG < a.n ? row0 + u * RG : a.n - 1;
                dst.scale[u][s] = load_scale(a.scales, row * gpr + ((li + s * L) >> 1));
            }
    };
    auto load_res = [&](uint32_t unit) -> float {
        const uint32_t row = (unit * U + (li >> (log_l - log_u))) * RG + rr;
        return residual && row < a.n ? residual[row] : 0.0f;
    };

    Unit A, B;
    RowValues rv;
    fetch_row<M>(a.x + (size_t)token * a.k, a.norm, a.k, rv);
    load(A, count ? wave : (full_units ? full_units - 1 : 0));
    __shared__ __attribute__((aligned(16))) Act8Lds lds;
    block_encode8<M>(rv, a.k, a.eps, lds);
    Act8 X[S];
#pragma unroll
    for (int s = 0; s < S; ++s) load_act8<Fmt8::Q5>(lds, li + s * L, X[s]);
    float resA = count ? load_res(wave) : 0.0f, resB = 0.0f;

    auto process = [&](const Unit &src, float res, uint32_t unit) __attribute__((always_inline)) {
        // The unit's bytes into this wavefront's LDS (its reads of the
        // previous unit came before, in program order).
#pragma unroll
        for (int m = 0; m < NWQ; ++m)
            if (lane + 64 * m < P) wl[lane + 64 * m] = src.w[m];
        const uint8_t *lb = reinterpret_cast<const uint8_t *>(wl);
        float acc[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const uint32_t c = li + s * L;
                const uint8_t *g = lb + (u * RG + rr) * row_bytes + (c >> 1) * 40u;
                Slice8<Fmt8::Q5> sl;
                sl.lo0 = *reinterpret_cast<const u32x2 *>(g + (c & 1u) * 16u);
                sl.lo1 = *reinterpret_cast<const u32x2 *>(g + (c & 1u) * 16u + 8u);
                sl.hi = *reinterpret_cast<const uint32_t *>(g + 32u + (c & 1u) * 4u);
                const float part = b8_slice_dot(sl, X[s]) * (dev::f16_bits_to_f32(src.scale[u][s]) * X[s].mult);
                acc[u] = s == 0 ? part : acc[u] + part;
            }
        }
        const float total = reduce_rows<U, L>(acc, lane);
        const bool writer = (li & ((L >> log_u) - 1)) == 0;
        const uint32_t row = (unit * U + (li >> (log_l - log_u))) * RG + rr;
        if (a.pairs) {
            const float partner = __shfl_down(total, RG > 1 ? L : (L >> log_u), kWave);
            if (writer && (row & 1u) == 0 && row < a.n) out[row >> 1] = silu_mul(total, partner);
        } else if (writer && row < a.n) {
            out[row] = res + total;
        }
    };

    uint32_t i = 0;
    for (; i + 1 < count; i += 2) {
        const uint32_t ua = wave + i * nwaves, ub = ua + nwaves;
        load(B, ub);
        resB = load_res(ub);
        process(A, resA, ua);
        const uint32_t un = i + 2 < count ? ub + nwaves : ub;
        load(A, un);
        resA = load_res(un);
        process(B, resB, ub);
    }
    if (i < count) process(A, resA, wave + i * nwaves);
    if (full_units < units && full_units % nwaves == wave) {
        load(B, full_units);
        process(B, load_res(full_units), full_units);
    }
}

// Any K up to the LDS encoding's 6144: one wavefront per row (per row pair
// with pairs), lanes striding over the row's slices.
template <Fmt8 F, Src M>
__global__ __launch_bounds__(256) void gemv_b8_generic_kernel(const GemvB8Args a) {
    const int lane = threadIdx.x & 63;
    const uint32_t wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const uint32_t nwaves = (gridDim.x * blockDim.x) >> 6;
    const uint32_t token = blockIdx.y;
    const uint32_t gpr = a.k >> 6;
    const uint32_t row_bytes = b8_row_bytes<F>(gpr);
    __shared__ __attribute__((aligned(16))) Act8Lds lds;
    RowValues rv;
    fetch_row<M>(a.x + (size_t)token * a.k, a.norm, a.k, rv);
    block_encode8<M>(rv, a.k, a.eps, lds);
    float *out = a.out + (size_t)token * (a.pairs ? a.n / 2 : a.n);
    const float *residual = a.residual ? a.residual + (size_t)token * a.n : nullptr;
    const uint32_t per = a.pairs ? 2u : 1u;
    for (uint32_t first = wave * per; first < a.n; first += nwaves * per) {
        float tot[2] = {0.0f, 0.0f};
        for (uint32_t r = 0; r < per; ++r) {
            float acc = 0.0f;
            for (uint32_t c = lane; c < a.t; c += 64) {
                Act8 x;
                load_act8<F>(lds, c, x);
                const Slice8<F> sl = load_slice8<F>(a, first + r, c, row_bytes, gpr);
                acc += b8_slice_dot(sl, x) * (dev::f16_bits_to_f32(sl.scale) * x.mult);
            }
            tot[r] = dev::wave_sum(acc);
        }
        if (lane == 0) {
            if (a.pairs) out[first >> 1] = silu_mul(tot[0], tot[1]);
            else out[first] = (residual ? residual[first] : 0.0f) + tot[0];
        }
    }
}

uint32_t gcd_u32(uint32_t a, uint32_t b) {
    while (b) {
        const uint32_t t = a % b;
        a = b;
        b = t;
    }
    return a;
}

// At most this many blocks (of four wavefronts) per compute unit: fewer
// concurrent streams keep HBM pages open.
constexpr int kBlocksPerCu = 4;
// Row groups per unit for the one-slice q4 kernels (the common shapes).
constexpr int kUnitRows = 4;

// Units each wavefront takes at least, when the kernel forms its own
// activations (that prologue is paid once per wavefront).
int min_units_per_wave() { return 1; }

// Blocks of 256 threads of `kernel` resident per compute unit (at most
// kBlocksPerCu), from the occupancy of that kernel, asked once per kernel.
int resident_blocks(const void *kernel) {
    static std::mutex lock;
    static std::unordered_map<const void *, int> known;
    std::lock_guard<std::mutex> guard(lock);
    auto it = known.find(kernel);
    if (it != known.end()) return it->second;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 256, 0) != hipSuccess || per_cu <= 0) {
        (void)hipGetLastError();
        per_cu = 4;
    }
    const int resident = per_cu < kBlocksPerCu ? per_cu : kBlocksPerCu;
    known.emplace(kernel, resident);
    return resident;
}

// Blocks to launch: every unit covered, no more blocks than can be resident
// at once (each wave then walks its share of the units).
template <typename Kernel>
unsigned grid_blocks(Kernel kernel, uint32_t units, int cus, uint32_t per_wave = 1) {
    const int resident = resident_blocks(reinterpret_cast<const void *>(kernel));
    uint32_t blocks = (units + 4 * per_wave - 1) / (4 * per_wave);
    uint32_t limit = (uint32_t)(cus > 0 ? cus : 256) * (uint32_t)resident;
    // At most 4096 wavefronts: with rows * 4096 < 2^32 (checked by the
    // launcher) the kernels' wave * units products stay within 32 bits.
    if (limit > 1024) limit = 1024;
    if (blocks > limit) blocks = limit;
    if (blocks == 0) blocks = 1;
    return blocks;
}

// Launches the kernel (or, with `blocks`, only reports its grid's width).
template <int S, int L, int U, Src M>
hipError_t launch_q4(hipStream_t s, int cus, GemvQ4Args args, uint32_t tokens, uint32_t *blocks) {
    args.row_groups = (args.n + (64 / L) - 1) / (64 / L);
    const uint32_t units = (args.row_groups + U - 1) / U;
    auto kernel = gemv_q4_kernel<S, L, U, M>;
    const uint32_t per_wave = M == Src::Digits ? 1u : (uint32_t)min_units_per_wave();
    const uint32_t grid = grid_blocks(kernel, units, cus, per_wave);
    if (blocks) {
        *blocks = grid;
        return hipSuccess;
    }
    kernel<<<dim3(grid, tokens), 256, 0, s>>>(args);
    return hipGetLastError();
}

template <Src M>
hipError_t dispatch_q4(hipStream_t s, int cus, const GemvQ4Args &args, uint32_t tokens, uint32_t S, uint32_t L,
                       bool &done, uint32_t *blocks = nullptr) {
    done = true;
    if constexpr (M == Src::Embed) {
        // One stretch of activations per thread: rows of K <= 2048.
        if (S == 1 && L == 64) return launch_q4<1, 64, kUnitRows, M>(s, cus, args, tokens, blocks);
        if (S == 1 && L == 32) return launch_q4<1, 32, kUnitRows, M>(s, cus, args, tokens, blocks);
        if (S == 1 && L == 16) return launch_q4<1, 16, kUnitRows, M>(s, cus, args, tokens, blocks);
        if (S == 1 && L == 8) return launch_q4<1, 8, 4, M>(s, cus, args, tokens, blocks);
    } else {
        if (S == 1 && L == 64) return launch_q4<1, 64, kUnitRows, M>(s, cus, args, tokens, blocks);
        if (S == 1 && L == 32) return launch_q4<1, 32, kUnitRows, M>(s, cus, args, tokens, blocks);
        if (S == 1 && L == 16) return launch_q4<1, 16, kUnitRows, M>(s, cus, args, tokens, blocks);
        if (S == 1 && L == 8) return launch_q4<1, 8, 4, M>(s, cus, args, tokens, blocks);
        if (S == 1 && L == 4) return launch_q4<1, 4, 4, M>(s, cus, args, tokens, blocks);
        if (S == 1 && L == 2) return launch_q4<1, 2, 2, M>(s, cus, args, tokens, blocks);
        if (S == 2 && L == 64) return launch_q4<2, 64, 4, M>(s, cus, args, tokens, blocks);
        if (S == 3 && L == 64) return launch_q4<3, 64, 2, M>(s, cus, args, tokens, blocks);
        if (S == 3 && L == 32) return launch_q4<3, 32, 2, M>(s, cus, args, tokens, blocks);
        if (S == 3 && L == 16) return launch_q4<3, 16, 2, M>(s, cus, args, tokens, blocks);
        if (S == 3 && L == 2) return launch_q4<3, 2, 2, M>(s, cus, args, tokens, blocks);
    }
    done = false;
    return hipSuccess;
}

// Shapes with a templated kernel: one, two or three slices per lane, a data
// plane below 4 GiB and few enough units for 32-bit unit arithmetic.
bool fused_shape(uint32_t rows, uint32_t cols, uint32_t &S, uint32_t &L) {
    const uint32_t T = cols / 32;
    L = gcd_u32(T, 64);
    S = T / L;
    const bool small = (uint64_t)rows * (cols / 2) < (1ull << 32) && (uint64_t)rows * 4096ull < (1ull << 32);
    const bool built = (S == 1 && (L == 64 || L == 32 || L == 16 || L == 8 || L == 4 || L == 2)) ||
                       (S == 2 && L == 64) || (S == 3 && (L == 64 || L == 32 || L == 16 || L == 2));
    return small && built;
}

}  // namespace

size_t q4_digit_bytes(uint32_t tokens, uint32_t cols) {
    const size_t chunks = (size_t)tokens * (cols / 32);
    return chunks * dev::kChunkWords * 4 + chunks * 4 + 256;
}

bool gemv_q4_fused_supported(uint32_t rows, uint32_t cols) {
    uint32_t S, L;
    return fused_shape(rows, cols, S, L);
}

bool gemv_q4_source_supported(int mode, uint32_t rows, uint32_t cols) {
    uint32_t S, L;
    if (!fused_shape(rows, cols, S, L)) return false;
    if (mode == GemvInput::Embed)
        return cols <= 2048 && S == 1 && (L == 64 || L == 32 || L == 16 || L == 8);
    return true;
}

hipError_t launch_prep_q4(hipStream_t s, const float *x, uint32_t tokens, uint32_t cols, void *digits) {
    const uint32_t total8 = tokens * (cols / 8);
    const size_t chunks = (size_t)tokens * (cols / 32);
    uint32_t *words = static_cast<uint32_t *>(digits);
    float *mult = reinterpret_cast<float *>(words + chunks * dev::kChunkWords);
    prep_q4_kernel<<<(total8 + 255) / 256, 256, 0, s>>>(x, total8, words, mult);
    return hipGetLastError();
}

namespace {

// Fills the kernel's arguments and launches it (with `blocks`, only reports
// the grid's width).
hipError_t q4_src(hipStream_t s, int cus, const GemvInput &in, const Matrix &w, uint32_t tokens, float *out,
                  const float *residual, uint32_t *blocks) {
    if (in.pairs && (w.rows & 1u)) return hipErrorInvalidValue;
    if (in.arg_value && (in.pairs || residual || !in.arg_index)) return hipErrorInvalidValue;
    if (in.mode == GemvInput::Embed) {
        const Matrix *e = in.embed;
        if (!e || e->cols != w.cols || w.cols > 2048 || !in.norm || !in.tokens || !in.rows || !in.row_flags ||
            !in.embed_out || !in.pos || !in.rope_cos || !in.rope_sin || !in.rope_now || 2 * in.rope_half > 256 ||
            (e->format != QWH_FORMAT_Q4 && e->format != QWH_FORMAT_Q5 && e->format != QWH_FORMAT_Q8))
            return hipErrorInvalidValue;
    }
    GemvQ4Args args{};
    const uint32_t T = w.cols / 32;
    args.scales = reinterpret_cast<const uint16_t *>(w.scales);
    args.data = w.data;
    args.out = out;
    args.residual = residual;
    args.n = w.rows;
    args.k = w.cols;
    args.t = T;
    args.x = in.x;
    args.norm = in.norm;
    args.eps = in.eps;
    args.pairs = in.pairs ? 1u : 0u;
    if (in.mode == GemvInput::Digits) {
        const size_t chunks = (size_t)tokens * T;
        args.words = static_cast<const uint32_t *>(in.digits);
        args.mult = reinterpret_cast<const float *>(args.words + chunks * dev::kChunkWords);
    }
    if (in.embed) {
        args.tokens = in.tokens;
        args.embed_format = in.embed->format;
        args.embed_scales = reinterpret_cast<const uint16_t *>(in.embed->scales);
        args.embed_data = in.embed->data;
    }
    args.rows = in.rows;
    args.row_flags = in.row_flags;
    args.hidden_out = in.embed_out;
    args.pos = in.pos;
    args.rope_cos = in.rope_cos;
    args.rope_sin = in.rope_sin;
    args.rope_half = in.rope_half;
    args.rope_now = in.rope_now;
    args.arg_value = in.arg_value;
    args.arg_index = in.arg_index;
    uint32_t S = 0, L = 0;
    const bool fused = fused_shape(w.rows, w.cols, S, L);
    bool done = false;
    hipError_t err = hipSuccess;
    if (fused) {
        switch (in.mode) {
        case GemvInput::Digits: err = dispatch_q4<Src::Digits>(s, cus, args, tokens, S, L, done, blocks); break;
        case GemvInput::F32: err = dispatch_q4<Src::F32>(s, cus, args, tokens, S, L, done, blocks); break;
        case GemvInput::RmsNorm: err = dispatch_q4<Src::RmsNorm>(s, cus, args, tokens, S, L, done, blocks); break;
        case GemvInput::Embed: err = dispatch_q4<Src::Embed>(s, cus, args, tokens, S, L, done, blocks); break;
        }
    }
    if (done) return err;
    if (in.mode != GemvInput::Digits || (in.pairs && residual) || in.arg_value) return hipErrorNotSupported;
    args.row_groups = w.rows;
    const uint32_t grid = grid_blocks(gemv_q4_generic_kernel, w.rows, cus);
    if (blocks) {
        *blocks = grid;
        return hipSuccess;
    }
    gemv_q4_generic_kernel<<<dim3(grid, tokens), 256, 0, s>>>(args);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemv_q4_src(hipStream_t s, int cus, const GemvInput &in, const Matrix &w, uint32_t tokens,
                              float *out, const float *residual) {
    return q4_src(s, cus, in, w, tokens, out, residual, nullptr);
}

uint32_t gemv_q4_partials(int cus, const Matrix &w, const GemvInput &in) {
    uint32_t blocks = 0;
    if (q4_src(nullptr, cus, in, w, 1, nullptr, nullptr, &blocks) != hipSuccess) return 0;
    return blocks;
}

hipError_t launch_gemv_q4(hipStream_t s, int cus, const void *digits, const Matrix &w, uint32_t tokens,
                          float *out, const float *residual) {
    GemvInput in{};
    in.mode = GemvInput::Digits;
    in.digits = digits;
    return launch_gemv_q4_src(s, cus, in, w, tokens, out, residual);
}

#define QWH_GEMV8_CASE(S_, L_, U_)                                                                 \
    if (S == S_ && L == L_ && small_plane) {                                                       \
        args.row_groups = (args.n + (64 / L_) - 1) / (64 / L_);                                    \
        const uint32_t units = (args.row_groups + U_ - 1) / U_;                                    \
        auto kernel = gemv_q8_kernel<S_, L_, U_>;                                                  \
        kernel<<<dim3(grid_blocks(kernel, units, cus), tokens), 256, 0, s>>>(args);                \
        return hipGetLastError();                                                                  \
    }

hipError_t launch_gemv_q8(hipStream_t s, int cus, const float *x, const Matrix &w, uint32_t tokens,
                          float *out, const float *residual) {
    GemvQ8Args args{};
    const uint32_t T = w.cols / 16;
    args.x = x;
    args.scales = reinterpret_cast<const uint16_t *>(w.scales);
    args.data = w.data;
    args.out = out;
    args.residual = residual;
    args.n = w.rows;
    args.k = w.cols;
    args.t = T;
    const uint32_t L = gcd_u32(T, 64);
    const uint32_t S = T / L;
    const bool small_plane = (uint64_t)w.rows * w.cols < (1ull << 32) && (uint64_t)w.rows * 4096ull < (1ull << 32);
    QWH_GEMV8_CASE(1, 64, 4)
    QWH_GEMV8_CASE(1, 32, 4)
    QWH_GEMV8_CASE(1, 16, 4)
    QWH_GEMV8_CASE(1, 8, 4)
    QWH_GEMV8_CASE(1, 4, 4)
    QWH_GEMV8_CASE(2, 64, 2)
    QWH_GEMV8_CASE(3, 64, 2)
    QWH_GEMV8_CASE(3, 16, 2)
    args.row_groups = w.rows;
    gemv_q8_generic_kernel<<<dim3(grid_blocks(gemv_q8_generic_kernel, w.rows, cus), tokens), 256, 0, s>>>(args);
    return hipGetLastError();
}

bool gemv_b8_supported(int format, uint32_t rows, uint32_t cols) {
    // The activations are encoded into LDS (at most kMaxChunks chunks), and
    // the kernels address the data plane with 32-bit offsets.
    const uint64_t per_group = format == QWH_FORMAT_Q5 ? 40 : format == QWH_FORMAT_Q8 ? 64 : 0;
    return per_group && cols % 64 == 0 && cols / 32 <= (uint32_t)kMaxChunks &&
           (uint64_t)rows * (cols / 64) * per_group < (1ull << 32) && (uint64_t)rows * 4096ull < (1ull << 32);
}

namespace {

template <Fmt8 F, Src M>
hipError_t dispatch_b8(hipStream_t s, int cus, GemvB8Args args, uint32_t tokens) {
    const uint32_t L = gcd_u32(args.t, 64);
    const uint32_t S = args.t / L;
    // q5 planes on 16-byte boundaries, up to 32768 rows: the staged form
    // (whole pieces). Measured on one box: the 1.7B q5 batch-1 step
    // 0.975-0.977 -> 0.965-0.966 ms; the 0.6B lm_head shape [151936 x 1024]
    // 22.8-23.1 us without it, 23.1-24.1 us with it, so longer matrices keep
    // the per-lane loads.
    const bool staged = F == Fmt8::Q5 && ((uintptr_t)args.data & 15u) == 0 && args.n <= 32768u;
#define QWH_GEMV_B8_CASE(S_, L_, U_)                                                               \
    if (S == S_ && L == L_) {                                                                      \
        args.row_groups = (args.n + (64 / L_) - 1) / (64 / L_);                                    \
        const uint32_t units = (args.row_groups + U_ - 1) / U_;                                    \
        if constexpr (F == Fmt8::Q5)                                                               \
            if (staged) {                                                                          \
                auto kernel = gemv_q5_staged_kernel<S_, L_, U_, M>;                                \
                kernel<<<dim3(grid_blocks(kernel, units, cus), tokens), 256, 0, s>>>(args);        \
                return hipGetLastError();                                                          \
            }                                                                                      \
        auto kernel = gemv_b8_kernel<F, S_, L_, U_, M>;                                            \
        kernel<<<dim3(grid_blocks(kernel, units, cus), tokens), 256, 0, s>>>(args);                \
        return hipGetLastError();                                                                  \
    }
    QWH_GEMV_B8_CASE(1, 64, 4)
    QWH_GEMV_B8_CASE(1, 32, 4)
    QWH_GEMV_B8_CASE(1, 16, 4)
    QWH_GEMV_B8_CASE(1, 8, 4)
    QWH_GEMV_B8_CASE(2, 64, 2)
    QWH_GEMV_B8_CASE(3, 64, 2)
    QWH_GEMV_B8_CASE(3, 32, 2)
#undef QWH_GEMV_B8_CASE
    args.row_groups = args.n;
    auto kernel = gemv_b8_generic_kernel<F, M>;
    const uint32_t work = args.pairs ? args.n / 2 : args.n;
    kernel<<<dim3(grid_blocks(kernel, work, cus), tokens), 256, 0, s>>>(args);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemv_b8(hipStream_t s, int cus, const GemvInput &in, const Matrix &w, uint32_t tokens, float *out,
                          const float *residual) {
    if (!gemv_b8_supported(w.format, w.rows, w.cols)) return hipErrorNotSupported;
    if (in.mode != GemvInput::F32 && in.mode != GemvInput::RmsNorm) return hipErrorNotSupported;
    if (in.pairs && ((w.rows & 1u) || residual)) return hipErrorInvalidValue;
    GemvB8Args args{};
    args.x = in.x;
    args.norm = in.norm;
    args.eps = in.eps;
    args.scales = reinterpret_cast<const uint16_t *>(w.scales);
    args.data = w.data;
    args.out = out;
    args.residual = residual;
    args.n = w.rows;
    args.k = w.cols;
    args.t = w.cols / 32;
    args.pairs = in.pairs ? 1u : 0u;
    const bool rms = in.mode == GemvInput::RmsNorm;
    if (w.format == QWH_FORMAT_Q5)
        return rms ? dispatch_b8<Fmt8::Q5, Src::RmsNorm>(s, cus, args, tokens)
                   : dispatch_b8<Fmt8::Q5, Src::F32>(s, cus, args, tokens);
    return rms ? dispatch_b8<Fmt8::Q8, Src::RmsNorm>(s, cus, args, tokens)
               : dispatch_b8<Fmt8::Q8, Src::F32>(s, cus, args, tokens);
}

}  // namespace qwh
