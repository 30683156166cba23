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
// decode_attention_q8.wgsl:56, does not apply). The softmax runs in base 2
// (scores carry a factor log2(e), exponentials are exp2): the same weights.
//
// The decoder form also does the work decoder.zig:180-216 does between the
// q/k/v projection and the attention: per-head RMSNorm of q and k, RoPE at the
// new position, and the q8 append of the new key and value rows. The range
// kernel normalizes and rotates its query heads and attends to every row
// before the new one; the merge kernel (one workgroup per query head, a
// thread per dimension) forms the new key and value rows, stores them in the
// cache, and adds the new position's score and value to the merged state.
//
// Lane mapping of the range kernel: a head row of D codes is D/16 lanes of 16
// bytes ("lane group"); a wavefront scores 64/(D/16) positions per load. Each
// lane holds its 16 query values for every head of the group in registers.
#include <cfloat>

#include "attention_plan.h"
#include "common.h"
#include "device.h"

namespace qwh {
namespace {

constexpr float kNeg = -1.0e30f;
// Word 3 of a raw buffer resource (gfx9 family: 32-bit data format; the
// range check is on byte offsets, stride 0).
constexpr int kBufferWord3 = 0x00020000;  // running-max sentinel: finite, so exp2(kNeg - kNeg) is defined
constexpr float kLog2e = 1.44269504088896340736f;
constexpr int kWaves = (int)plan::kWaves;

struct AttnKernelArgs {
    const float *query;  // row of sequence b at query + b * query_stride; head h at h * D
    uint32_t query_stride;
    uint8_t *k_scales, *k_codes, *v_scales, *v_codes;
    const uint32_t *cached_dev;
    uint32_t cached, cached_bias;
    uint32_t rows;       // cache rows that may be read (>= every sequence's cached)
    uint32_t heads, kv_heads;
    uint32_t chunk;      // positions per workgroup
    uint32_t splits;
    uint64_t scale_stride, code_stride;
    float scaling;       // log2(e) / sqrt(D)
    float *partial;      // [batch][kv_heads][splits] records of R*D + 4*R floats
    float *out;          // [batch][heads][D]
    // Decoder form.
    const float *q_norm, *k_norm;
    const float *rope_now;  // [batch][D]: cos (D/2) then sin (D/2) of the new position
    float eps;
    // Optional digit-plane copy of the output (small-batch GEMV layout).
    uint8_t *digits;
    float *digit_mult;
    // Query rows as a K-split GEMV's partial sums (query_slices > 1): the
    // planes are query_plane floats apart and are summed in slice order.
    uint32_t query_slices;
    uint64_t query_plane;
    // Decoder form with the newest row already in the cache (a prefill):
    // the range kernels attend to it like any other row.
    uint32_t attend_newest;
};

constexpr uint32_t kMaxQuerySlices = 8;

// The partial values of query-row element `off`, one per slice (loads for
// slices past the count repeat the last one: they stay unconditional).
__device__ __forceinline__ void query_parts(const AttnKernelArgs &a, size_t off, float (&w)[kMaxQuerySlices]) {
#pragma unroll
    for (uint32_t s = 0; s < kMaxQuerySlices; ++s)
        w[s] = a.query[(size_t)(s < a.query_slices ? s : a.query_slices - 1) * a.query_plane + off];
}

// Their sum in slice order (the order of the GEMV's own slice reduce).
__device__ __forceinline__ float query_sum(const AttnKernelArgs &a, const float (&w)[kMaxQuerySlices]) {
    float v = w[0];
#pragma unroll
    for (uint32_t s = 1; s < kMaxQuerySlices; ++s)
        if (s < a.query_slices) v += w[s];
    return v;
}

// Element `off` of the query rows.
__device__ __forceinline__ float query_value(const AttnKernelArgs &a, size_t off) {
    if (a.query_slices <= 1) return a.query[off];
    float w[kMaxQuerySlices];
    query_parts(a, off, w);
    return query_sum(a, w);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

using dev::group_sum;

// math.rmsNormInPlace (math.zig:120-130) of one head row spread over the LPP
// lanes of a lane group (16 values per lane); `weight` holds this lane's 16
// weights.
template <int D>
__device__ __forceinline__ void rms_norm16(float (&x)[16], const float (&weight)[16], float eps) {
    constexpr int LPP = D / 16;
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) ss = __fadd_rn(ss, __fmul_rn(x[i], x[i]));
    ss = group_sum<LPP>(ss);
    const float inverse_rms = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)D), eps)));
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = __fmul_rn(__fmul_rn(x[i], inverse_rms), weight[i]);
}

// rotate_half RoPE (kernels.zig:495-527) with the tables' row for the
// position: the partner of dimension d < D/2 is d + D/2, held by lane
// sub ^ LPP/2. c[i], s[i] are the table entries of this lane's dimensions.
template <int D>
__device__ __forceinline__ void rope16(float (&x)[16], const float (&c)[16], const float (&s)[16], int sub) {
    constexpr int LPP = D / 16;
    const bool first = sub < LPP / 2;
    float y[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float partner = dev::xor_lane<LPP / 2>(x[i]);
        y[i] = first ? __fsub_rn(__fmul_rn(x[i], c[i]), __fmul_rn(partner, s[i]))
                     : __fadd_rn(__fmul_rn(x[i], c[i]), __fmul_rn(partner, s[i]));
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = y[i];
}

__device__ __forceinline__ void load16(const float *p, float (&v)[16]) {
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
        const float4 f = *reinterpret_cast<const float4 *>(p + i);
        v[i] = f.x; v[i + 1] = f.y; v[i + 2] = f.z; v[i + 3] = f.w;
    }
}

template <int R>
struct SoftmaxState {
    float m[R], l[R], acc[R][16];
};

// Online-softmax update by a block of NB scores per query head: the running
// maximum, the rescaled running sum and accumulator; w receives the block's
// weights exp2(score - max) (0 for invalid positions).
template <int R, int NB>
__device__ __forceinline__ void softmax_update(SoftmaxState<R> &st, const float (&score)[NB][R], const bool (&valid)[NB],
                                               float (&w)[NB][R]) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float bm = score[0][r];
#pragma unroll
        for (int nb = 1; nb < NB; ++nb) bm = fmaxf(bm, score[nb][r]);
        const float m_new = fmaxf(st.m[r], bm);
        const float alpha = fast_exp2(st.m[r] - m_new);
        float sum = 0.0f;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            w[nb][r] = valid[nb] ? fast_exp2(score[nb][r] - m_new) : 0.0f;
            sum += w[nb][r];
        }
        st.l[r] = st.l[r] * alpha + sum;
        st.m[r] = m_new;
#pragma unroll
        for (int i = 0; i < 16; ++i) st.acc[r][i] *= alpha;
    }
}

// f32 cache (kernels.zig:572-627 decodeAttentionStep): scores q . k per
// position over the LPP lanes of a lane group, values accumulated as they
// are.
template <int D, int R, int NB>
__device__ __forceinline__ void attend_f32(SoftmaxState<R> &st, const float (&q)[R][16], const float (&k)[NB][16],
                                           const float (&v)[NB][16], const bool (&valid)[NB], float scaling) {
    constexpr int LPP = D / 16;
    float score[NB][R];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float dot = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) dot = fmaf(k[nb][i], q[r][i], dot);
            const float part = group_sum<LPP>(dot);
            score[nb][r] = valid[nb] ? part * scaling : kNeg;
        }
    }
    float w[NB][R];
    softmax_update<R, NB>(st, score, valid, w);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int i = 0; i < 16; ++i) st.acc[r][i] = fmaf(w[nb][r], v[nb][i], st.acc[r][i]);
}

// ---- q8 range kernel: key scores on the matrix cores ----
//
// The scores of 16 positions against up to four query heads are one
// v_mfma_i32_16x16x64_i8 per 64-value scale group, on exact integers:
//   keys     the codes u - 128 as signed bytes (u ^ 0x80);
//   query    per head and group, x_int = rint(q * 2^(22-e)) with 2^e bounding
//            the group's largest |q| (|x_int| <= 2^22), as three signed
//            base-256 digit planes d0 + 256 d1 + 65536 d2, the encoding of the
//            small-batch GEMV's activations.
// Operand rows (A) are (head, plane) = 4 * head + plane (plane 3 is zero),
// operand columns (B) are positions, and both take the 64 group values in
// the same order (lane l: values 16 * (l / 16) .. +15), so the sum runs over
// the whole group. Lane l then holds the three plane sums of head l / 16 for
// position l % 16 ("score layout"); their combination times the group's f16
// key scale and 2^(e-22) is the group's share of the score
// sum_g scale_g * sum_{d in g} (u_d - 128) q_d (kernels.zig:727-735).
// Each plane sum is at most 64 * 128 * 128 = 2^20 in magnitude: the int32
// results are exact.
//
// The values are accumulated on the vector ALUs in the "value layout": a head
// row of D codes is D/16 lanes of 16 bytes (a lane group), each lane group
// takes kTile / (64 / (D/16)) consecutive positions of the wavefront's tile.
// The softmax weights cross from the score layout to the value layout
// through a wavefront-private LDS row per head. The running maximum of each
// head is one value for the whole wavefront (it is reduced over the 16
// positions of a block and read back as a scalar), so the accumulators of
// all lane groups share it, rescale by one scalar factor (skipped while the
// maximum stands still), and merge at the end by plain sums.

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kTile = (int)plan::kTile;    // positions per wavefront per iteration
constexpr int kTileBlocks = kTile / 16;   // 16-position MFMA blocks per tile

// LDS stores of this wavefront before its later LDS loads of other lanes'
// data (LDS operations of one wavefront complete in order; the fences keep
// the compiler from moving them across).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// 16 q8 codes as signed bytes u - 128.
__device__ __forceinline__ v4i signed_codes(const uint4 w) {
    v4i b;
    b.x = (int)(w.x ^ 0x80808080u);
    b.y = (int)(w.y ^ 0x80808080u);
    b.z = (int)(w.z ^ 0x80808080u);
    b.w = (int)(w.w ^ 0x80808080u);
    return b;
}

// Digit plane `plane` of x_int = rint(x * up) for 16 values (byte b of the
// result belongs to x[b]): (x_int + 0x808080) ^ 0x808080 holds the three
// signed digits as its bytes.
__device__ __forceinline__ v4i digit_plane16(const float *x, float up, int plane) {
    v4i out;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        uint32_t word = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const uint32_t u = (uint32_t)((int)__builtin_rintf(x[4 * w + b] * up) + 0x808080) ^ 0x808080u;
            word |= ((u >> (8 * plane)) & 0xffu) << (8 * b);
        }
        out[w] = (int)word;
    }
    return out;
}

// Sum over the lanes that hold the same 16-byte slice for other positions
// (lanes l ^ (k * LPP)).
template <int LPP>
__device__ __forceinline__ float sum_over_groups(float v) {
    if constexpr (LPP <= 4) v += dev::xor_lane<4>(v);
    if constexpr (LPP <= 8) v += dev::xor_lane<8>(v);
    if constexpr (LPP <= 16) v += dev::xor_lane<16>(v);
    return v + dev::xor_lane<32>(v);
}

// Maximum over the 16 lanes of a score-layout row (one head, 16 positions).
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dev::xor_lane<1>(v));
    v = fmaxf(v, dev::xor_lane<2>(v));
    v = fmaxf(v, dev::xor_lane<4>(v));
    return fmaxf(v, dev::xor_lane<8>(v));
}

__device__ __forceinline__ float lane_value(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Online-softmax merge of (m, l, acc) into a running (M, L, A).
__device__ __forceinline__ void merge_state(float &M, float &L, float4 &A, float m, float l, float4 v) {
    const float m_new = fmaxf(M, m);
    const float fa = fast_exp2(M - m_new);
    const float fb = fast_exp2(m - m_new);
    L = L * fa + l * fb;
    A.x = A.x * fa + v.x * fb;
    A.y = A.y * fa + v.y * fb;
    A.z = A.z * fa + v.z * fb;
    A.w = A.w * fa + v.w * fb;
    M = m_new;
}

// One step of the merge of the lane groups: lanes l and l ^ MASK combine
// their online-softmax states.
template <int MASK, int R>
__device__ __forceinline__ void merge_step(SoftmaxState<R> &st) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float m_o = dev::xor_lane<MASK>(st.m[r]);
        const float l_o = dev::xor_lane<MASK>(st.l[r]);
        const float m_new = fmaxf(st.m[r], m_o);
        const float a_self = fast_exp2(st.m[r] - m_new);
        const float a_other = fast_exp2(m_o - m_new);
        st.l[r] = st.l[r] * a_self + l_o * a_other;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float o = dev::xor_lane<MASK>(st.acc[r][i]);
            st.acc[r][i] = st.acc[r][i] * a_self + o * a_other;
        }
        st.m[r] = m_new;
    }
}

template <int LPP, int R>
__device__ __forceinline__ void merge_lane_groups(SoftmaxState<R> &st) {
    if constexpr (LPP <= 4) merge_step<4, R>(st);
    if constexpr (LPP <= 8) merge_step<8, R>(st);
    if constexpr (LPP <= 16) merge_step<16, R>(st);
    merge_step<32, R>(st);
}

// The end of a range kernel: the lanes of lane group 0 hold their wave's
// merged state for their slice (the lane groups already merged), and the
// waves merge in wave order through LDS into this range's (acc, m, l) record.
template <int D, int R>
__device__ __forceinline__ void write_range_record(const AttnKernelArgs &a, const SoftmaxState<R> &st, uint32_t b,
                                                   uint32_t kvh, uint32_t split, int wave, int sub, int group) {
    constexpr int REC = R * D + 4 * R;
    __shared__ float lds_acc[kWaves][R][D];
    __shared__ float lds_ml[kWaves][R][2];
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
            const float f = fast_exp2(lds_ml[w2][r][0] - M);
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

template <int D>
__device__ __forceinline__ void write_digits(const AttnKernelArgs &a, uint32_t b, uint32_t h, int col, float4 o);

// The range kernel. Early: the second tile's loads are issued before the
// query prologue too (a range of two tiles per wavefront then waits for
// memory once), at the cost of that tile's registers during the prologue.
template <int D, int R, bool Decoder, bool Early>
__device__ __forceinline__ void attention_range(const AttnKernelArgs &a) {
    constexpr int LPP = D / 16;              // value layout: lanes per position
    constexpr int PPW = 64 / LPP;            // value layout: lane groups per wave
    constexpr int NV = kTile / PPW;          // consecutive positions per lane group per tile
    constexpr int G = D / 64;                // scale groups per head
    constexpr int HS = (R + 3) / 4;          // MFMA row sets of four heads
    constexpr uint32_t kSpan = kTile * kWaves;
    static_assert(R <= PPW, "one lane group per head in the query prologue");
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int sub = lane % LPP;              // value layout: 16-byte slice of the head row
    const int group = lane / LPP;            // value layout: lane group
    const int n = lane & 15;                 // score layout: position in the block
    const int quarter = lane >> 4;           // score layout: head in the row set; operand value slice
    const uint32_t split = blockIdx.x;
    const uint32_t kvh = blockIdx.y;
    const uint32_t b = blockIdx.z;
    const uint32_t kv_width = a.kv_heads * D;
    const uint32_t gpr = kv_width / 64;
    const uint32_t begin = split * a.chunk;
    const uint16_t *k_scales = reinterpret_cast<const uint16_t *>(a.k_scales + b * a.scale_stride);
    const uint16_t *v_scales = reinterpret_cast<const uint16_t *>(a.v_scales + b * a.scale_stride);
    const uint8_t *k_codes = a.k_codes + b * a.code_stride;
    const uint8_t *v_codes = a.v_codes + b * a.code_stride;
    const uint32_t key_col = kvh * D + quarter * 16;   // + 64 g
    const uint32_t code_col = kvh * D + sub * 16;

    __shared__ float lds_q[R][D];
    __shared__ int lds_exp[R][G];
    // The values' products run on the matrix cores. Per wavefront, the
    // tile's value codes (signed bytes, [position][dimension], rows padded
    // by 16 bytes so a transposing read's eight rows fall on distinct
    // banks) and the weights' digit planes ([group][head * 4 + plane]
    // [position]; rows of plane 3 and of heads past R stay zero). The
    // range record's partial sums reuse the same bytes after the loop.
    constexpr int kVcRow = D + 16;
    constexpr int kVcBytes = kTile * kVcRow;
    constexpr int kPlBytes = G * 32 * kTile;
    constexpr int kMvWave = kVcBytes + kPlBytes;
    constexpr int kMvRecord = (kWaves * R * D + kWaves * R * 2) * 4;
    constexpr int kMvBytes = kWaves * kMvWave > kMvRecord ? kWaves * kMvWave : kMvRecord;
    __shared__ __attribute__((aligned(16))) uint8_t lds_mv[kMvBytes];
    uint8_t *vcl = lds_mv + wave * kMvWave;
    uint8_t *pll = vcl + kVcBytes;

    // A tile: the wavefront's kTile positions from base + wave * kTile; keys
    // and key and value scales in the score layout, values in the value
    // layout, scales as raw f16 bits.
    struct Tile {
        uint4 kc[kTileBlocks][G];
        uint32_t ks[kTileBlocks][G];
        uint4 vc[NV];
        uint32_t vsc[kTileBlocks][G];
    };
    // Every load is unconditional, so all of a tile's loads are in flight
    // together. Plain form: tiles are read through buffer resources that
    // start at the tile's first row and end at `limit` (the allocated rows,
    // or `end` once the position is known): a lane's byte offsets within a
    // tile are the same for every tile and the resource is scalar
    // arithmetic, so a tile costs no vector address arithmetic, and a row at
    // or past `limit` reads zeros through the hardware range check without
    // touching memory (batch 16 and batch 8 at 4096 / 8192 positions: 31.3
    // -> 29.3 us and 31.5 -> 28.9 us). Decoder form: global loads with each
    // row at or past `limit` clamped to row limit - 1 (one cached line) and
    // masked when the tile is used; the buffer form measured 1-3 % slower
    // there (33.4 against 32.3 us per batch-16 layer, same box).
    uint32_t key_off[kTileBlocks], kscale_off[kTileBlocks], val_off[NV];
#pragma unroll
    for (int blk = 0; blk < kTileBlocks; ++blk) {
        const uint32_t rel = wave * kTile + 16 * blk + n;
        key_off[blk] = rel * kv_width + key_col;
        kscale_off[blk] = (rel * gpr + kvh * G) * 2;
    }
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        const uint32_t rel = wave * kTile + NV * group + v;
        val_off[v] = rel * kv_width + code_col;
    }
    auto load_tile_global = [&](Tile &t, uint32_t base, uint32_t limit) {
        const uint32_t first = base + wave * kTile;
#pragma unroll
        for (int blk = 0; blk < kTileBlocks; ++blk) {
            const uint32_t p = first + 16 * blk + n;
            const uint32_t row = p < limit ? p : limit - 1;
#pragma unroll
            for (int g = 0; g < G; ++g)
                t.kc[blk][g] = *reinterpret_cast<const uint4 *>(k_codes + (size_t)row * kv_width + key_col + 64 * g);
            if constexpr (G == 2) {
                // Both groups' scales of a row in one 4-byte load each.
                const uint32_t kk = *reinterpret_cast<const uint32_t *>(k_scales + (size_t)row * gpr + kvh * G);
                const uint32_t vv = *reinterpret_cast<const uint32_t *>(v_scales + (size_t)row * gpr + kvh * G);
                t.ks[blk][0] = kk & 0xffffu;
                t.ks[blk][1] = kk >> 16;
                t.vsc[blk][0] = vv & 0xffffu;
                t.vsc[blk][1] = vv >> 16;
            } else {
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    t.ks[blk][g] = k_scales[(size_t)row * gpr + kvh * G + g];
                    t.vsc[blk][g] = v_scales[(size_t)row * gpr + kvh * G + g];
                }
            }
        }
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const uint32_t p = first + NV * group + v;
            const uint32_t row = p < limit ? p : limit - 1;
            t.vc[v] = *reinterpret_cast<const uint4 *>(v_codes + (size_t)row * kv_width + code_col);
        }
    };
    auto load_tile = [&](Tile &t, uint32_t base_in, uint32_t limit) {
        if constexpr (Decoder) {
            load_tile_global(t, base_in, limit);
            return;
        }
        // (Scalars: the resources must be uniform.)
        const uint32_t base = __builtin_amdgcn_readfirstlane(base_in);
        const uint32_t rows = __builtin_amdgcn_readfirstlane(base < limit ? limit - base : 0u);
        const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t *>(k_codes + (size_t)base * kv_width), 0, (int)(rows * kv_width), kBufferWord3);
        const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t *>(v_codes + (size_t)base * kv_width), 0, (int)(rows * kv_width), kBufferWord3);
        const __amdgpu_buffer_rsrc_t ksr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t *>(k_scales + (size_t)base * gpr), 0, (int)(rows * gpr * 2), kBufferWord3);
        const __amdgpu_buffer_rsrc_t vsr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t *>(v_scales + (size_t)base * gpr), 0, (int)(rows * gpr * 2), kBufferWord3);
#pragma unroll
        for (int blk = 0; blk < kTileBlocks; ++blk) {
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const v4i c = __builtin_bit_cast(
                    v4i, __builtin_amdgcn_raw_buffer_load_b128(kr, (int)key_off[blk] + 64 * g, 0, 0));
                t.kc[blk][g] = make_uint4((uint32_t)c.x, (uint32_t)c.y, (uint32_t)c.z, (uint32_t)c.w);
            }
            if constexpr (G == 2) {
                const uint32_t kk = __builtin_amdgcn_raw_buffer_load_b32(ksr, (int)kscale_off[blk], 0, 0);
                const uint32_t vv = __builtin_amdgcn_raw_buffer_load_b32(vsr, (int)kscale_off[blk], 0, 0);
                t.ks[blk][0] = kk & 0xffffu;
                t.ks[blk][1] = kk >> 16;
                t.vsc[blk][0] = vv & 0xffffu;
                t.vsc[blk][1] = vv >> 16;
            } else {
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    t.ks[blk][g] = __builtin_amdgcn_raw_buffer_load_b16(ksr, (int)kscale_off[blk] + 2 * g, 0, 0);
                    t.vsc[blk][g] = __builtin_amdgcn_raw_buffer_load_b16(vsr, (int)kscale_off[blk] + 2 * g, 0, 0);
                }
            }
        }
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const v4i c = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(vr, (int)val_off[v], 0, 0));
            t.vc[v] = make_uint4((uint32_t)c.x, (uint32_t)c.y, (uint32_t)c.z, (uint32_t)c.w);
        }
    };

    // The query slices, norm weights and RoPE row are requested first and the
    // first tile right after them, before the sequence's position is known
    // (in the decoder it is a device value, one memory round trip away):
    // every allocated row is readable, and rows past the position are
    // dropped once it has arrived. Loads complete in issue order, so the
    // query prologue waits only for its own values while the tile is in
    // flight (tile first measured 1-3 % slower at batch 1). Lane group r < R
    // of wavefront 0 takes query head r.
    const bool prologue = wave == 0 && group < R;
    const int qh = prologue ? group : 0;
    const float *row = a.query + (size_t)b * a.query_stride;
    float q[16];
    // Sliced query rows: the workgroup sums the R heads' values, QP per
    // thread, into LDS once the tile loads are out.
    constexpr int QP = (R * D + 255) / 256;
    const bool sliced = a.query_slices > 1;
    float qparts[QP][kMaxQuerySlices];
    if (sliced) {
#pragma unroll
        for (int i = 0; i < QP; ++i) {
            const uint32_t idx = threadIdx.x + 256 * i < (uint32_t)(R * D) ? threadIdx.x + 256 * i : 0;
            query_parts(a, (size_t)b * a.query_stride + kvh * R * D + idx, qparts[i]);
        }
    } else {
        load16(row + (kvh * R + qh) * D + sub * 16, q);
    }
    float wq[16], rc[16], rs[16];
    if (Decoder) {
        const int j0 = (sub % (LPP / 2)) * 16;
        load16(a.q_norm + sub * 16, wq);
        load16(a.rope_now + (size_t)b * D + j0, rc);
        load16(a.rope_now + (size_t)b * D + D / 2 + j0, rs);
    }
    Tile cur, nxt;
    load_tile(cur, begin, a.rows);
    if constexpr (Early) load_tile(nxt, begin + kSpan, a.rows);
    if (sliced) {
#pragma unroll
        for (int i = 0; i < QP; ++i)
            if (threadIdx.x + 256 * i < (uint32_t)(R * D))
                (&lds_q[0][0])[threadIdx.x + 256 * i] = query_sum(a, qparts[i]);
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 16; ++i) q[i] = lds_q[qh][sub * 16 + i];
    }
    const uint32_t cached = a.cached_dev ? a.cached_dev[b] + a.cached_bias : a.cached;
    // The decoder form leaves the newest row (cached - 1) to the merge kernel.
    const uint32_t attended = Decoder && !a.attend_newest ? cached - 1 : cached;
    uint32_t end = begin + a.chunk;
    if (end > attended) end = attended;

    if (begin >= cached) return;  // no record: the merge reads ranges below cached only
    if (Decoder) {
        rms_norm16<D>(q, wq, a.eps);
        rope16<D>(q, rc, rs, sub);
    }
    // The query heads and each group's exponent into LDS.
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(q[i]));
    amax = fmaxf(amax, dev::xor_lane<1>(amax));
    amax = fmaxf(amax, dev::xor_lane<2>(amax));
    if (prologue) {
#pragma unroll
        for (int i = 0; i < 16; i += 4)
            *reinterpret_cast<float4 *>(&lds_q[qh][sub * 16 + i]) = make_float4(q[i], q[i + 1], q[i + 2], q[i + 3]);
        if (sub % 4 == 0) lds_exp[qh][sub / 4] = dev::chunk_exponent(amax);
    }
    __syncthreads();
    // Operand rows of this lane: head 4 hs + n / 4, plane n % 4; its values
    // 64 g + 16 quarter .. +15. Score-layout multipliers: head 4 hs + quarter.
    v4i qa[HS][G];
    float qm[HS][G];
#pragma unroll
    for (int hs = 0; hs < HS; ++hs) {
        const int ra = 4 * hs + n / 4, plane = n % 4;
        const int rq = 4 * hs + quarter;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            v4i op = {0, 0, 0, 0};
            if (ra < R && plane < 3)
                op = digit_plane16(&lds_q[ra][64 * g + 16 * quarter], __builtin_ldexpf(1.0f, 22 - lds_exp[ra][g]), plane);
            qa[hs][g] = op;
            qm[hs][g] = rq < R ? __builtin_ldexpf(a.scaling, lds_exp[rq][g] - 22) : 0.0f;
        }
    }

    // Running state: m (the same in every lane of a head's score row), the
    // lane's share of l (score layout), acc (the product layout: dimension
    // 32 j + lane % 32 of head 2 q + lane / 32 in acc[j][q], the wavefront's
    // whole sum).
    constexpr int NB = D / 32;               // 32-dimension blocks of a head row
    constexpr int HQ = (R + 1) / 2;          // heads per lane in the product layout
    float m[HS], l[HS];
    float acc[NB][HQ];
#pragma unroll
    for (int hs = 0; hs < HS; ++hs) {
        m[hs] = kNeg;
        l[hs] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int q = 0; q < HQ; ++q) acc[j][q] = 0.0f;
    // Zero digit planes: plane 3 and heads past R are never written.
#pragma unroll
    for (int g = 0; g < G; ++g) *reinterpret_cast<v4i *>(pll + g * 32 * kTile + 16 * lane) = v4i{0, 0, 0, 0};

    // The tile's values, acc += sum over its positions of (w * scale) *
    // (u - 128), on the matrix cores. The weights times their position's
    // value scale, per head and 64-dimension group, become three signed
    // digit planes of x = rint(w s 2^(22 - e)) (e from the largest of the
    // head's tile values, so x <= 2^22; zero weights, rows past `end`, give
    // zero digits whatever their codes); one v_mfma_i32_32x32x32_i8 per 32
    // dimensions multiplies [head * 4 + plane][position] digits by the codes
    // [position][dimension] (read transposed from LDS, eight positions of a
    // dimension per lane and read), and the three planes' integer sums are
    // combined as in the scores: (c0 + 256 c1) + 65536 c2, times 2^(e - 22).
    auto use_values_mfma = [&](const Tile &t, const float (&wv)[HS][kTileBlocks], const bool (&valid)[kTileBlocks],
                               const float (&alpha)[R]) __attribute__((always_inline)) {
        // The tile's codes (signed) into this wavefront's rows.
#pragma unroll
        for (int v = 0; v < NV; ++v)
            *reinterpret_cast<v4i *>(vcl + (NV * group + v) * kVcRow + sub * 16) = signed_codes(t.vc[v]);
        float mult[HS][G];
#pragma unroll
        for (int hs = 0; hs < HS; ++hs) {
            const int rq = 4 * hs + quarter;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float W[kTileBlocks];
                float wmax = 0.0f;
#pragma unroll
                for (int blk = 0; blk < kTileBlocks; ++blk) {
                    W[blk] = valid[blk] ? wv[hs][blk] * dev::f16_bits_to_f32((uint16_t)t.vsc[blk][g]) : 0.0f;
                    wmax = fmaxf(wmax, W[blk]);
                }
                wmax = row16_max(wmax);
                // wmax < 2^e (e kept above -100 so 2^(22 - e) stays finite).
                int e = (int)((__builtin_bit_cast(uint32_t, wmax) >> 23) & 0xffu) - 126;
                e = e < -100 ? -100 : e;
                const float up = wmax > 0.0f ? __builtin_ldexpf(1.0f, 22 - e) : 0.0f;
                mult[hs][g] = wmax > 0.0f ? __builtin_ldexpf(1.0f, e - 22) : 0.0f;
                if (rq < R) {
#pragma unroll
                    for (int blk = 0; blk < kTileBlocks; ++blk) {
                        const uint32_t y = (uint32_t)((int)__builtin_rintf(W[blk] * up) + 0x808080) ^ 0x808080u;
                        uint8_t *dst = pll + (g * 32 + rq * 4) * kTile + 16 * blk + n;
                        dst[0] = (uint8_t)y;
                        dst[kTile] = (uint8_t)(y >> 8);
                        dst[2 * kTile] = (uint8_t)(y >> 16);
                    }
                }
            }
        }
        wave_lds_sync();
        // Rescale to the new maxima (head 2 q + lane / 32 of acc[.][q]).
        bool moved = false;
#pragma unroll
        for (int r = 0; r < R; ++r) moved |= alpha[r] != 1.0f;
        if (moved) {
#pragma unroll
            for (int q = 0; q < HQ; ++q) {
                const float al = lane < 32 ? alpha[2 * q] : alpha[2 * q + 1 < R ? 2 * q + 1 : 2 * q];
#pragma unroll
                for (int j = 0; j < NB; ++j) acc[j][q] *= al;
            }
        }
        v4i A[G];
#pragma unroll
        for (int g = 0; g < G; ++g)
            A[g] = *reinterpret_cast<const v4i *>(pll + (g * 32 + (lane & 31)) * kTile + 16 * (lane >> 5));
        float mh[HQ][G];
#pragma unroll
        for (int q = 0; q < HQ; ++q)
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const int h0 = 2 * q, h1 = 2 * q + 1;
                const float m0 = lane_value(mult[h0 / 4][g], 16 * (h0 % 4));
                const float m1 = h1 < R ? lane_value(mult[h1 / 4][g], 16 * (h1 % 4)) : 0.0f;
                mh[q][g] = lane < 32 ? m0 : m1;
            }
        // Transposed code reads: in each 16-lane group, lane i takes byte i
        // of the eight 16-byte rows that lanes (2 b, 2 b + 1) address.
        const int ti = lane & 15;
        const uint8_t *src0 = vcl + (16 * (lane >> 5) + (ti >> 1)) * kVcRow + 16 * ((lane >> 4) & 1) + 8 * (ti & 1);
        const v16i zero16 = {};
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int g = j / 2;
            const uint8_t *src = src0 + 32 * j;
            const v2i b0 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i *)src);
            const v2i b1 =
                __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i *)(src + 8 * kVcRow));
            const v4i B = {b0.x, b0.y, b1.x, b1.y};
            const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[g], B, zero16, 0, 0, 0);
#pragma unroll
            for (int q = 0; q < HQ; ++q) {
                const float val = (float)(c[4 * q] + 256 * c[4 * q + 1]) + 65536.0f * (float)c[4 * q + 2];
                acc[j][q] = fmaf(val, mh[q][g], acc[j][q]);
            }
        }
        wave_lds_sync();
    };

    // Rows below `end` take part; the others (possibly never written, so
    // their bits are arbitrary) get no weight and a zero value scale.
    auto use_tile = [&](const Tile &t, uint32_t base) {
        const uint32_t first = base + wave * kTile;
        const v4i zero = {0, 0, 0, 0};
        float s[HS][kTileBlocks];
        bool valid[kTileBlocks];
#pragma unroll
        for (int blk = 0; blk < kTileBlocks; ++blk) {
            valid[blk] = first + 16 * blk + n < end;
            v4i kb[G];
            float ks[G];
#pragma unroll
            for (int g = 0; g < G; ++g) {
                kb[g] = signed_codes(t.kc[blk][g]);
                ks[g] = dev::f16_bits_to_f32((uint16_t)t.ks[blk][g]);
            }
#pragma unroll
            for (int hs = 0; hs < HS; ++hs) {
                float sc = 0.0f;
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const v4i c = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa[hs][g], kb[g], zero, 0, 0, 0);
                    const float dot = (float)(c.x + 256 * c.y) + 65536.0f * (float)c.z;
                    sc = fmaf(dot, qm[hs][g] * ks[g], sc);
                }
                s[hs][blk] = valid[blk] ? sc : kNeg;
            }
        }
        // Online softmax per head over the tile; the weights stay in
        // registers, the rescale factors become scalars.
        float alpha[R];
        float wv[HS][kTileBlocks];
#pragma unroll
        for (int hs = 0; hs < HS; ++hs) {
            float mx = s[hs][0];
#pragma unroll
            for (int blk = 1; blk < kTileBlocks; ++blk) mx = fmaxf(mx, s[hs][blk]);
            const float m_new = fmaxf(m[hs], row16_max(mx));
            const float al = fast_exp2(m[hs] - m_new);
            float sum = 0.0f;
#pragma unroll
            for (int blk = 0; blk < kTileBlocks; ++blk) {
                const float w = valid[blk] ? fast_exp2(s[hs][blk] - m_new) : 0.0f;
                sum += w;
                wv[hs][blk] = w;
            }
            l[hs] = l[hs] * al + sum;
            m[hs] = m_new;
#pragma unroll
            for (int k = 0; k < 4 && 4 * hs + k < R; ++k) alpha[4 * hs + k] = lane_value(al, 16 * k);
        }
        use_values_mfma(t, wv, valid, alpha);
    };

    // Double buffered, two tiles per trip: the next tile's loads are in
    // flight while the current one is scored and accumulated. The loads are
    // issued whether or not the tile holds positions (past `end` they read
    // zeros without a memory access, or one cached line): a load under a
    // branch makes the compiler's wait for the current tile also wait for
    // the loads issued after it. The scheduling barriers keep the work on the current tile
    // (which waits for its data) from moving above the next tile's loads.
    if (begin < end) {
        if constexpr (!Early) {
            load_tile(nxt, begin + kSpan, end);
            __builtin_amdgcn_sched_barrier(0);
        }
        use_tile(cur, begin);
        if (begin + kSpan < end) {
            load_tile(cur, begin + 2 * kSpan, end);
            __builtin_amdgcn_sched_barrier(0);
            use_tile(nxt, begin + kSpan);
            for (uint32_t base = begin + 2 * kSpan; base < end; base += 2 * kSpan) {
                load_tile(nxt, base + kSpan, end);
                __builtin_amdgcn_sched_barrier(0);
                use_tile(cur, base);
                if (base + kSpan >= end) break;
                load_tile(cur, base + 2 * kSpan, end);
                __builtin_amdgcn_sched_barrier(0);
                use_tile(nxt, base + kSpan);
            }
        }
    }

    // The wave's state: the lane groups share each head's maximum, so their
    // accumulators merge by sums; l is summed over the head's score row.
    SoftmaxState<R> st;
#pragma unroll
    for (int hs = 0; hs < HS; ++hs) {
        float lsum = l[hs];
        lsum += dev::xor_lane<1>(lsum);
        lsum += dev::xor_lane<2>(lsum);
        lsum += dev::xor_lane<4>(lsum);
        lsum += dev::xor_lane<8>(lsum);
#pragma unroll
        for (int k = 0; k < 4 && 4 * hs + k < R; ++k) {
            st.m[4 * hs + k] = lane_value(m[hs], 16 * k);
            st.l[4 * hs + k] = lane_value(lsum, 16 * k);
        }
    }
    {
        // Every wavefront is past its loop: the tile bytes hold the record's
        // parts now. Each lane's sums are its wavefront's whole sums.
        __syncthreads();
        float *part = reinterpret_cast<float *>(lds_mv);  // [kWaves][R][D]
        float *ml = part + kWaves * R * D;                  // [kWaves][R][2]
#pragma unroll
        for (int q = 0; q < HQ; ++q) {
            const int h = 2 * q + (lane >> 5);
            if (h < R)
#pragma unroll
                for (int j = 0; j < NB; ++j) part[(wave * R + h) * D + 32 * j + (lane & 31)] = acc[j][q];
        }
        if (lane == 0)
#pragma unroll
            for (int r = 0; r < R; ++r) {
                ml[(wave * R + r) * 2 + 0] = st.m[r];
                ml[(wave * R + r) * 2 + 1] = st.l[r];
            }
        __syncthreads();
        if (Decoder && a.attend_newest && a.splits == 1) {
            // A prefill row's only range: the merge would read this one
            // record, so the output (and the next GEMV's digits) is formed
            // here, as the merge forms it: A * (1 / L), four dimensions per
            // thread, whole 16-lane rows per 64-value group.
            for (int t = threadIdx.x; t < R * D / 4; t += blockDim.x) {
                const int r = t / (D / 4), col = t % (D / 4);
                float M = ml[r * 2];
#pragma unroll
                for (int w = 1; w < kWaves; ++w) M = fmaxf(M, ml[(w * R + r) * 2]);
                float L = 0.0f;
                float4 A = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
                for (int w = 0; w < kWaves; ++w) {
                    const float f = fast_exp2(ml[(w * R + r) * 2] - M);
                    L += ml[(w * R + r) * 2 + 1] * f;
                    const float4 p = *reinterpret_cast<const float4 *>(&part[(w * R + r) * D + 4 * col]);
                    A.x += p.x * f;
                    A.y += p.y * f;
                    A.z += p.z * f;
                    A.w += p.w * f;
                }
                const float inv = 1.0f / L;
                const float4 o = make_float4(A.x * inv, A.y * inv, A.z * inv, A.w * inv);
                const uint32_t h = kvh * R + r;
                *reinterpret_cast<float4 *>(a.out + ((size_t)b * a.heads + h) * D + 4 * col) = o;
                if (a.digits) write_digits<D>(a, b, h, col, o);
            }
            return;
        }
        constexpr int REC = R * D + 4 * R;
        float *rec = a.partial + (((size_t)b * a.kv_heads + kvh) * a.splits + split) * REC;
        for (int idx = threadIdx.x; idx < R * D; idx += blockDim.x) {
            const int r = idx / D;
            const int d = idx % D;
            float M = ml[r * 2];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) M = fmaxf(M, ml[(w * R + r) * 2]);
            float L = 0.0f, A = 0.0f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                const float f = fast_exp2(ml[(w * R + r) * 2] - M);
                L += ml[(w * R + r) * 2 + 1] * f;
                A += part[(w * R + r) * D + d] * f;
            }
            rec[idx] = A;
            if (d == 0) {
                rec[R * D + 4 * r + 0] = M;
                rec[R * D + 4 * r + 1] = L;
            }
        }
    }
}

// The q8 range kernel. Forms that fit three wavefronts per SIMD (168
// registers) without spilling are compiled for that occupancy (and load the
// second tile after the prologue); the others, and every form when the grid
// is at most one workgroup per CU (occupancy does not matter there), use
// the full register budget and load both tiles first.
template <int D, int R, bool Decoder>
constexpr bool kThreeWaves = R <= 2 && (D == 64 || (D == 128 && Decoder));

template <int D, int R, bool Decoder>
__global__ __launch_bounds__(256) void attention_kernel(const AttnKernelArgs a) {
    attention_range<D, R, Decoder, true>(a);
}

template <int D, int R, bool Decoder>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void attention_kernel3(const AttnKernelArgs a) {
    attention_range<D, R, Decoder, false>(a);
}


// The range kernel over an f32 cache (kernels.zig:572-627): the same lane
// mapping (a lane group of D/16 lanes per position, 16 dimensions per lane,
// four 16-byte loads per row), blocks of two positions per lane group (an f32
// row is four times a q8 row's registers), and the same records.
template <int D, int R, bool Decoder>
__global__ __launch_bounds__(256) void attention_f32_kernel(const AttnKernelArgs a) {
    constexpr int LPP = D / 16;
    constexpr int PPW = 64 / LPP;
    constexpr int STEP = PPW * kWaves;
    constexpr int NB = 2;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int sub = lane % LPP;
    const int group = lane / LPP;
    const uint32_t split = blockIdx.x;
    const uint32_t kvh = blockIdx.y;
    const uint32_t b = blockIdx.z;
    const uint32_t kv_width = a.kv_heads * D;
    const uint32_t begin = split * a.chunk;
    const float *keys = reinterpret_cast<const float *>(a.k_codes + b * a.code_stride);
    const float *values = reinterpret_cast<const float *>(a.v_codes + b * a.code_stride);
    const uint32_t col = kvh * D + sub * 16;
    constexpr uint32_t kSpan = STEP * NB;

    struct Block {
        float4 k[NB][4], v[NB][4];
    };
    // Unconditional loads, rows at or past `limit` clamped (as the q8 kernel).
    auto load_block = [&](Block &blk, uint32_t base, uint32_t limit) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const uint32_t p = base + nb * STEP + wave * PPW + group;
            const uint32_t row = p < limit ? p : limit - 1;
            const float4 *kp = reinterpret_cast<const float4 *>(keys + (size_t)row * kv_width + col);
            const float4 *vp = reinterpret_cast<const float4 *>(values + (size_t)row * kv_width + col);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                blk.k[nb][i] = kp[i];
                blk.v[nb][i] = vp[i];
            }
        }
    };
    // Rows past `end` get no score and contribute zero values.
    auto use_block = [&](SoftmaxState<R> &st, const float (&q)[R][16], const Block &blk, uint32_t base,
                         uint32_t end) {
        bool valid[NB];
        float k[NB][16], v[NB][16];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            valid[nb] = base + nb * STEP + wave * PPW + group < end;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                k[nb][4 * i] = blk.k[nb][i].x; k[nb][4 * i + 1] = blk.k[nb][i].y;
                k[nb][4 * i + 2] = blk.k[nb][i].z; k[nb][4 * i + 3] = blk.k[nb][i].w;
                v[nb][4 * i] = valid[nb] ? blk.v[nb][i].x : 0.0f; v[nb][4 * i + 1] = valid[nb] ? blk.v[nb][i].y : 0.0f;
                v[nb][4 * i + 2] = valid[nb] ? blk.v[nb][i].z : 0.0f; v[nb][4 * i + 3] = valid[nb] ? blk.v[nb][i].w : 0.0f;
            }
        }
        attend_f32<D, R, NB>(st, q, k, v, valid, a.scaling);
    };
    Block cur, nxt;
    load_block(cur, begin, a.rows);
    const float *row = a.query + (size_t)b * a.query_stride;
    float q[R][16];
    if (a.query_slices > 1) {
        // Sliced query rows: summed by the workgroup into LDS first.
        __shared__ float lds_q32[R * D];
        for (uint32_t idx = threadIdx.x; idx < (uint32_t)(R * D); idx += blockDim.x)
            lds_q32[idx] = query_value(a, (size_t)b * a.query_stride + kvh * R * D + idx);
        __syncthreads();
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int i = 0; i < 16; ++i) q[r][i] = lds_q32[r * D + sub * 16 + i];
    } else {
#pragma unroll
        for (int r = 0; r < R; ++r) load16(row + (kvh * R + r) * D + sub * 16, q[r]);
    }
    float wq[16], rc[16], rs[16];
    if (Decoder) {
        const int j0 = (sub % (LPP / 2)) * 16;
        load16(a.q_norm + sub * 16, wq);
        load16(a.rope_now + (size_t)b * D + j0, rc);
        load16(a.rope_now + (size_t)b * D + D / 2 + j0, rs);
    }
    const uint32_t cached = a.cached_dev ? a.cached_dev[b] + a.cached_bias : a.cached;
    const uint32_t attended = Decoder && !a.attend_newest ? cached - 1 : cached;
    uint32_t end = begin + a.chunk;
    if (end > attended) end = attended;
    if (begin >= cached) return;
    if (Decoder) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            rms_norm16<D>(q[r], wq, a.eps);
            rope16<D>(q[r], rc, rs, sub);
        }
    }
    SoftmaxState<R> st;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        st.m[r] = kNeg;
        st.l[r] = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) st.acc[r][i] = 0.0f;
    }
    for (uint32_t base = begin; base < end; base += kSpan) {
        const bool more = base + kSpan < end;
        if (more) load_block(nxt, base + kSpan, end);
        use_block(st, q, cur, base, end);
        if (more) cur = nxt;
    }
    merge_lane_groups<LPP, R>(st);
    write_range_record<D, R>(a, st, b, kvh, split, wave, sub, group);
}

// Sum over the D threads 0..D-1 (D/64 whole wavefronts) of the workgroup,
// in a fixed order; `slots` is LDS scratch of D/64 floats. Every thread of
// the workgroup must call it.
template <int D>
__device__ __forceinline__ float head_sum(float v, float *slots) {
    const int t = threadIdx.x;
    v = dev::wave_sum(v);
    if (t < D && (t & 63) == 0) slots[t >> 6] = v;
    __syncthreads();
    float s = slots[0];
#pragma unroll
    for (int w = 1; w < D / 64; ++w) s += slots[w];
    __syncthreads();
    return s;
}

// The output row of sequence b, head h, dimensions 4 col .. 4 col + 3, also
// as the small-batch GEMV's activation digits (the layout and arithmetic of
// prep_batch_kernel for F32 input, so the GEMV sees the same integers): per
// 64-value group (16 consecutive threads), x_int = rint(x * 2^(22-e)) with
// 2^e bounding the group's largest |x|, three signed base-256 digit planes;
// within each 8-value block the even columns' bytes come first, then the odd
// ones'. Threads 0 .. D/4 - 1 (whole rows of 16 lanes) call it together.
template <int D>
__device__ __forceinline__ void write_digits(const AttnKernelArgs &a, uint32_t b, uint32_t h, int col, float4 o) {
    constexpr uint32_t kTokens = 16, kPlane = kTokens * 64, kGroup = 3 * kPlane;
    float amax = fmaxf(fmaxf(fabsf(o.x), fabsf(o.y)), fmaxf(fabsf(o.z), fabsf(o.w)));
    amax = fmaxf(amax, dev::xor_lane<1>(amax));
    amax = fmaxf(amax, dev::xor_lane<2>(amax));
    amax = fmaxf(amax, dev::xor_lane<4>(amax));
    amax = fmaxf(amax, dev::xor_lane<8>(amax));
    const int ex = dev::chunk_exponent(amax);
    const float up = __builtin_ldexpf(1.0f, 22 - ex);
    const float v[4] = {o.x, o.y, o.z, o.w};
    uint32_t u[4], pu[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        u[i] = (uint32_t)((int)__builtin_rintf(v[i] * up) + 0x808080) ^ 0x808080u;
        pu[i] = __builtin_bit_cast(uint32_t, dev::xor_lane<1>(__builtin_bit_cast(float, u[i])));
    }
    // Columns k = 0..3 of the 8-value block are the even thread's, 4..7 its
    // partner's: the even thread writes the even columns, the odd one the
    // odd columns.
    const bool odd = col & 1;
    const uint32_t c0 = odd ? pu[1] : u[0], c1 = odd ? pu[3] : u[2], c2 = odd ? u[1] : pu[0], c3 = odd ? u[3] : pu[2];
    const uint32_t gpr = a.heads * D / 64;
    const uint32_t g = (h * D + 4 * col) / 64;
    const uint32_t tile = b / kTokens, tt = b % kTokens;
    uint8_t *dst = a.digits + ((size_t)tile * gpr + g) * kGroup + tt * 64 + ((4 * col) % 64 / 8) * 8 + (odd ? 4 : 0);
#pragma unroll
    for (int p = 0; p < 3; ++p) {
        const int sh = 8 * p;
        *reinterpret_cast<uint32_t *>(dst + p * kPlane) = ((c0 >> sh) & 0xffu) | (((c1 >> sh) & 0xffu) << 8) |
                                                           (((c2 >> sh) & 0xffu) << 16) | (((c3 >> sh) & 0xffu) << 24);
    }
    if (col % 16 == 0) a.digit_mult[((size_t)tile * gpr + g) * kTokens + tt] = __builtin_ldexpf(1.0f, ex - 22);
}

// out[h][d] = sum_s e^{m_s - M} acc_s[d] / sum_s e^{m_s - M} l_s over the
// ranges that hold positions, in range order, for query head h = kvh * R + r.
// Thread t takes four dimensions (column t % COLS) of the ranges congruent to
// t / COLS; the SL partial merges are then combined in order. The first
// kFirst ranges of each thread are loaded before the sequence's position is
// known (every record of the scratch is readable; those of ranges past the
// position are skipped).
//
// Decoder form: thread d < D also forms dimension d of the new position
// (cached - 1): q and k get RMSNorm and RoPE, k and v are quantized to q8 per
// 64-value group (one wavefront per group) -- or, with an f32 cache, kept as
// they are -- and stored by the first query head of the kv head, and the new
// row's score and (dequantized) value join the merge last.
template <int D, int R, bool Decoder, bool F32C>
__global__ __launch_bounds__(256) void attention_combine_kernel(const AttnKernelArgs a) {
    constexpr int REC = R * D + 4 * R;
    constexpr int COLS = D / 4;
    constexpr int SL = 256 / COLS;
    constexpr int kFirst = 8;
    static_assert(D <= 256, "one thread per dimension");
    const uint32_t h = blockIdx.x;
    const uint32_t b = blockIdx.y;
    const uint32_t kvh = h / R;
    const int r = (int)(h % R);
    const int t = threadIdx.x;
    const int col = t % COLS;
    const int j = t / COLS;
    const float *recs = a.partial + ((size_t)b * a.kv_heads + kvh) * a.splits * REC;
    float m[kFirst], l[kFirst];
    float4 v[kFirst];
    // Unconditional loads (a range past the last reads the last record and is
    // dropped below), so that all kFirst of them are in flight together.
#pragma unroll
    for (int q = 0; q < kFirst; ++q) {
        const uint32_t s = j + q * SL < a.splits ? j + q * SL : a.splits - 1;
        const float *rec = recs + (size_t)s * REC;
        m[q] = rec[R * D + 4 * r];
        l[q] = rec[R * D + 4 * r + 1];
        v[q] = *reinterpret_cast<const float4 *>(rec + r * D + 4 * col);
    }
    const uint32_t kv_width = a.kv_heads * D;
    float qx = 0.0f, kx = 0.0f, vx = 0.0f, wq = 0.0f, wk = 0.0f, rope_c = 0.0f, rope_s = 0.0f;
    if (Decoder && t < D) {
        const size_t base = (size_t)b * a.query_stride;
        qx = query_value(a, base + h * D + t);
        kx = query_value(a, base + a.heads * D + kvh * D + t);
        vx = query_value(a, base + a.heads * D + kv_width + kvh * D + t);
        wq = a.q_norm[t];
        wk = a.k_norm[t];
        rope_c = a.rope_now[(size_t)b * D + (t % (D / 2))];
        rope_s = a.rope_now[(size_t)b * D + D / 2 + (t % (D / 2))];
    }
    const uint32_t cached = a.cached_dev ? a.cached_dev[b] + a.cached_bias : a.cached;
    const uint32_t needed = (cached + a.chunk - 1) / a.chunk;
    const uint32_t used = needed < a.splits ? needed : a.splits;
    float M = kNeg, L = 0.0f;
    float4 A = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int q = 0; q < kFirst; ++q)
        if (j + q * SL < used) merge_state(M, L, A, m[q], l[q], v[q]);
    for (uint32_t s = j + kFirst * SL; s < used; s += SL) {
        const float *rec = recs + (size_t)s * REC;
        merge_state(M, L, A, rec[R * D + 4 * r], rec[R * D + 4 * r + 1],
                    *reinterpret_cast<const float4 *>(rec + r * D + 4 * col));
    }
    __shared__ float lds_m[256], lds_l[256];
    __shared__ float4 lds_a[256];
    __shared__ float lds_qk[2][D];
    __shared__ float lds_v[D];
    __shared__ float lds_sum[D / 64];
    __shared__ float lds_score;
    lds_m[t] = M;
    lds_l[t] = L;
    lds_a[t] = A;

    if (Decoder) {
        // decoder.zig:180-216 for dimension t of the new position.
        const uint32_t newest = cached - 1;
        const float ssq = head_sum<D>(t < D ? __fmul_rn(qx, qx) : 0.0f, lds_sum);
        const float ssk = head_sum<D>(t < D ? __fmul_rn(kx, kx) : 0.0f, lds_sum);
        if (t < D) {
            const float inv_q = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ssq, (float)D), a.eps)));
            const float inv_k = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ssk, (float)D), a.eps)));
            lds_qk[0][t] = __fmul_rn(__fmul_rn(qx, inv_q), wq);
            lds_qk[1][t] = __fmul_rn(__fmul_rn(kx, inv_k), wk);
        }
        __syncthreads();
        float qr = 0.0f, code_k = 0.0f, scale_k = 0.0f;
        if (t < D) {
            const int half = D / 2;
            const float c = rope_c, s = rope_s;
            const float qn = lds_qk[0][t], kn = lds_qk[1][t];
            const float qp = lds_qk[0][t ^ half], kp = lds_qk[1][t ^ half];
            qr = t < half ? __fsub_rn(__fmul_rn(qn, c), __fmul_rn(qp, s)) : __fadd_rn(__fmul_rn(qn, c), __fmul_rn(qp, s));
            const float kr = t < half ? __fsub_rn(__fmul_rn(kn, c), __fmul_rn(kp, s))
                                      : __fadd_rn(__fmul_rn(kn, c), __fmul_rn(kp, s));
            const size_t pos_codes = (size_t)newest * kv_width + kvh * D + t;
            if constexpr (F32C) {
                // decoder.zig:77-83: the f32 cache stores the rows as they are.
                code_k = kr;
                scale_k = 1.0f;
                lds_v[t] = vx;
                if (r == 0) {
                    reinterpret_cast<float *>(a.k_codes + b * a.code_stride)[pos_codes] = kr;
                    reinterpret_cast<float *>(a.v_codes + b * a.code_stride)[pos_codes] = vx;
                }
            } else {
                // quantizeRow(.q8): this wavefront is one 64-value group.
                const uint16_t kbits = dev::f32_to_f16_bits(__fdiv_rn(dev::wave_max(fabsf(kr)), 128.0f));
                const uint16_t vbits = dev::f32_to_f16_bits(__fdiv_rn(dev::wave_max(fabsf(vx)), 128.0f));
                scale_k = dev::f16_bits_to_f32(kbits);
                const float scale_v = dev::f16_bits_to_f32(vbits);
                const int ck = dev::quantize_one(kr, scale_k, -128, 127);
                const int cv = dev::quantize_one(vx, scale_v, -128, 127);
                code_k = (float)ck;
                lds_v[t] = (float)cv * scale_v;
                if (r == 0) {
                    const size_t pos_scales = (size_t)newest * (kv_width / 64) + kvh * (D / 64) + (t >> 6);
                    a.k_codes[b * a.code_stride + pos_codes] = (uint8_t)(ck + 128);
                    a.v_codes[b * a.code_stride + pos_codes] = (uint8_t)(cv + 128);
                    if ((t & 63) == 0) {
                        reinterpret_cast<uint16_t *>(a.k_scales + b * a.scale_stride)[pos_scales] = kbits;
                        reinterpret_cast<uint16_t *>(a.v_scales + b * a.scale_stride)[pos_scales] = vbits;
                    }
                }
            }
        }
        // Score of the new position (kernels.zig:727-735): per group
        // scale * sum (u - 128) q, summed over groups, times the scaling
        // (f32 cache: k . q times the scaling, kernels.zig:603-608).
        const float part = dev::wave_sum(t < D ? code_k * qr : 0.0f);
        if (t < D && (t & 63) == 0) lds_sum[t >> 6] = part * scale_k;
        __syncthreads();
        if (t == 0) {
            float sc = lds_sum[0];
#pragma unroll
            for (int w = 1; w < D / 64; ++w) sc += lds_sum[w];
            lds_score = sc * a.scaling;
        }
    }
    __syncthreads();
    if (t < COLS) {
        for (int k = 1; k < SL; ++k) merge_state(M, L, A, lds_m[k * COLS + col], lds_l[k * COLS + col], lds_a[k * COLS + col]);
        if (Decoder) {
            const float4 vn = make_float4(lds_v[4 * col], lds_v[4 * col + 1], lds_v[4 * col + 2], lds_v[4 * col + 3]);
            merge_state(M, L, A, lds_score, 1.0f, vn);
        }
        const float inv = 1.0f / L;
        const float4 o = make_float4(A.x * inv, A.y * inv, A.z * inv, A.w * inv);
        *reinterpret_cast<float4 *>(a.out + ((size_t)b * a.heads + h) * D + 4 * col) = o;
        if (a.digits) write_digits<D>(a, b, h, col, o);
    }
}

// decoder.zig:180-216 and :77-105 for a run of new positions of one
// sequence (a prefill): for position i and kv head blockIdx.x, the key row
// (from the q | k | v rows, or the sum of their K-slice partials) gets
// RMSNorm and RoPE at its position (rope row i), and the key and value rows
// are stored at cache row first + i -- q8 per 64-value group (one wavefront
// per group), or as they are in an f32 cache. The arithmetic of the step's
// merge kernel, one thread per dimension.
template <int D, bool F32C>
__global__ __launch_bounds__(D) void prefill_append_kernel(const AttnKernelArgs a, uint32_t first) {
    const uint32_t kvh = blockIdx.x;
    const uint32_t i = blockIdx.y;
    const int t = threadIdx.x;
    const uint32_t kv_width = a.kv_heads * D;
    const size_t base = (size_t)i * a.query_stride;
    const float kx = query_value(a, base + a.heads * D + kvh * D + t);
    const float vx = query_value(a, base + a.heads * D + kv_width + kvh * D + t);
    const float wk = a.k_norm[t];
    const float rope_c = a.rope_now[(size_t)i * D + (t % (D / 2))];
    const float rope_s = a.rope_now[(size_t)i * D + D / 2 + (t % (D / 2))];
    __shared__ float lds_k[D];
    __shared__ float lds_sum[D / 64];
    const float ssk = head_sum<D>(__fmul_rn(kx, kx), lds_sum);
    const float inv_k = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ssk, (float)D), a.eps)));
    lds_k[t] = __fmul_rn(__fmul_rn(kx, inv_k), wk);
    __syncthreads();
    const int half = D / 2;
    const float kn = lds_k[t], kp = lds_k[t ^ half];
    const float kr = t < half ? __fsub_rn(__fmul_rn(kn, rope_c), __fmul_rn(kp, rope_s))
                              : __fadd_rn(__fmul_rn(kn, rope_c), __fmul_rn(kp, rope_s));
    const uint32_t row = first + i;
    const size_t pos_codes = (size_t)row * kv_width + kvh * D + t;
    if constexpr (F32C) {
        reinterpret_cast<float *>(a.k_codes)[pos_codes] = kr;
        reinterpret_cast<float *>(a.v_codes)[pos_codes] = vx;
    } else {
        const uint16_t kbits = dev::f32_to_f16_bits(__fdiv_rn(dev::wave_max(fabsf(kr)), 128.0f));
        const uint16_t vbits = dev::f32_to_f16_bits(__fdiv_rn(dev::wave_max(fabsf(vx)), 128.0f));
        const int ck = dev::quantize_one(kr, dev::f16_bits_to_f32(kbits), -128, 127);
        const int cv = dev::quantize_one(vx, dev::f16_bits_to_f32(vbits), -128, 127);
        a.k_codes[pos_codes] = (uint8_t)(ck + 128);
        a.v_codes[pos_codes] = (uint8_t)(cv + 128);
        if ((t & 63) == 0) {
            const size_t pos_scales = (size_t)row * (kv_width / 64) + kvh * (D / 64) + (t >> 6);
            reinterpret_cast<uint16_t *>(a.k_scales)[pos_scales] = kbits;
            reinterpret_cast<uint16_t *>(a.v_scales)[pos_scales] = vbits;
        }
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

// ---- Any head shape (the range kernels' lane mapping needs head_dim 64,
// 128 or 256): kernels.zig:697-767 (q8) and :572-627 (f32) for every
// head_dim (a multiple of 64 for q8) up to kGenericMaxDim and every ratio of
// heads to kv heads. One workgroup per (query head, sequence) walks the
// positions 256 at a time: thread i scores position base + i over the whole
// head row (the q8 form per 64-value group: scale times the sum of
// (u - 128) q), the workgroup keeps an online softmax in base 2 (the running
// maximum and sum), and each thread accumulates the dimensions
// i, i + 256, ... over the block's positions with the weights from LDS.
constexpr uint32_t kGenericMaxDim = 1024;

__device__ __forceinline__ float block_max_256(float v, float *lds) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(lds[0], lds[1]), fmaxf(lds[2], lds[3]));
}

template <bool F32C>
__global__ __launch_bounds__(256) void attention_generic_kernel(const AttnKernelArgs a, uint32_t head_dim) {
    constexpr int kDims = kGenericMaxDim / 256;  // dimensions per thread
    __shared__ float q[kGenericMaxDim];
    __shared__ float w[256];
    __shared__ float red[4];
    const uint32_t h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
    const uint32_t D = head_dim;
    const uint32_t kvh = h / (a.heads / a.kv_heads);
    const uint32_t kv_width = a.kv_heads * D;
    const uint32_t gpr = kv_width / 64;
    const float *query = a.query + (size_t)b * a.query_stride + (size_t)h * D;
    for (uint32_t d = tid; d < D; d += 256) q[d] = query[d];
    __syncthreads();
    const uint8_t *k_codes = a.k_codes + b * a.code_stride;
    const uint8_t *v_codes = a.v_codes + b * a.code_stride;
    const uint16_t *k_scales = reinterpret_cast<const uint16_t *>(a.k_scales + b * a.scale_stride);
    const uint16_t *v_scales = reinterpret_cast<const uint16_t *>(a.v_scales + b * a.scale_stride);
    float acc[kDims];
#pragma unroll
    for (int j = 0; j < kDims; ++j) acc[j] = 0.0f;
    float m = kNeg, l = 0.0f;
    for (uint32_t base = 0; base < a.cached; base += 256) {
        const uint32_t p = base + tid;
        float s = kNeg;
        if (p < a.cached) {
            float dot = 0.0f;
            if constexpr (F32C) {
                const float *k = reinterpret_cast<const float *>(k_codes) + (size_t)p * kv_width + kvh * D;
                for (uint32_t d = 0; d < D; ++d) dot = fmaf(q[d], k[d], dot);
            } else {
                const uint8_t *k = k_codes + (size_t)p * kv_width + kvh * D;
                for (uint32_t g = 0; g < D / 64; ++g) {
                    float part = 0.0f;
                    for (uint32_t d = 0; d < 64; ++d) part = fmaf(q[64 * g + d], (float)((int)k[64 * g + d] - 128), part);
                    dot = fmaf(dev::f16_bits_to_f32(k_scales[(size_t)p * gpr + kvh * (D / 64) + g]), part, dot);
                }
            }
            s = dot * a.scaling;
        }
        const float m_new = fmaxf(m, block_max_256(s, red));
        const float e = p < a.cached ? fast_exp2(s - m_new) : 0.0f;
        const float alpha = fast_exp2(m - m_new);
        w[tid] = e;
        l = l * alpha + dev::block_sum_256(e, red);  // (its barriers also publish w)
        m = m_new;
        const uint32_t n = a.cached - base < 256 ? a.cached - base : 256;
#pragma unroll
        for (int j = 0; j < kDims; ++j) {
            const uint32_t d = tid + 256 * j;
            if (d >= D) break;
            float sum = 0.0f;
            for (uint32_t i = 0; i < n; ++i) {
                const size_t row = (size_t)(base + i) * kv_width + kvh * D;
                float v;
                if constexpr (F32C) {
                    v = reinterpret_cast<const float *>(v_codes)[row + d];
                } else {
                    v = (float)((int)v_codes[row + d] - 128) *
                        dev::f16_bits_to_f32(v_scales[(size_t)(base + i) * gpr + (kvh * D + d) / 64]);
                }
                sum = fmaf(w[i], v, sum);
            }
            acc[j] = acc[j] * alpha + sum;
        }
        __syncthreads();  // w is rewritten by the next block
    }
    const float inv = 1.0f / l;
    float *out = a.out + ((size_t)b * a.heads + h) * D;
#pragma unroll
    for (int j = 0; j < kDims; ++j) {
        const uint32_t d = tid + 256 * j;
        if (d < D) out[d] = acc[j] * inv;
    }
}

}  // namespace

size_t attention_scratch_bytes(int cus, const AttentionArgs &a) { return plan::scratch_bytes(cus, a); }

bool attention_generic_supported(uint32_t head_dim) { return head_dim >= 1 && head_dim <= kGenericMaxDim; }

bool attention_supported(uint32_t head_dim, uint32_t ratio) {
    return (head_dim == 64 && (ratio == 1 || ratio == 2 || ratio == 4)) ||
           (head_dim == 128 && (ratio == 1 || ratio == 2 || ratio == 4 || ratio == 8)) ||
           (head_dim == 256 && (ratio == 1 || ratio == 2));
}

// The range kernel and the merge. The decoder form's range kernel
// normalizes and rotates the queries; with k.attend_newest (a prefill, whose
// rows are all in the cache) the plain merge follows it.
template <int D, int R>
void launch_attention_pair(hipStream_t s, int cus, const AttnKernelArgs &k, bool decoder, bool f32, uint32_t splits,
                           uint32_t kv_heads, uint32_t heads, uint32_t batch) {
    const bool merge_new = decoder && !k.attend_newest;
    const dim3 ranges(splits, kv_heads, batch), merge(heads, batch);
    const bool sparse = (uint64_t)splits * kv_heads * batch <= (uint64_t)(cus > 0 ? cus : 256);
    if (f32) {
        if (decoder) {
            attention_f32_kernel<D, R, true><<<ranges, 256, 0, s>>>(k);
            if (merge_new) attention_combine_kernel<D, R, true, true><<<merge, 256, 0, s>>>(k);
            else attention_combine_kernel<D, R, false, true><<<merge, 256, 0, s>>>(k);
        } else {
            attention_f32_kernel<D, R, false><<<ranges, 256, 0, s>>>(k);
            attention_combine_kernel<D, R, false, true><<<merge, 256, 0, s>>>(k);
        }
    } else if (decoder) {
        bool launched = false;
        if constexpr (kThreeWaves<D, R, true>) {
            if (!sparse) {
                attention_kernel3<D, R, true><<<ranges, 256, 0, s>>>(k);
                launched = true;
            }
        }
        if (!launched) attention_kernel<D, R, true><<<ranges, 256, 0, s>>>(k);
        // A prefill whose rows each fit one range: the range kernel wrote
        // the output itself.
        if (k.attend_newest && splits == 1) return;
        if (merge_new) attention_combine_kernel<D, R, true, false><<<merge, 256, 0, s>>>(k);
        else attention_combine_kernel<D, R, false, false><<<merge, 256, 0, s>>>(k);
    } else {
        bool three = false;
        if constexpr (kThreeWaves<D, R, false>) {
            three = !sparse;
            if (three) attention_kernel3<D, R, false><<<ranges, 256, 0, s>>>(k);
        }
        if (!three) attention_kernel<D, R, false><<<ranges, 256, 0, s>>>(k);
        attention_combine_kernel<D, R, false, false><<<merge, 256, 0, s>>>(k);
    }
}

#define QWH_ATTN_CASE(D_, R_)                                                                       \
    if (a.head_dim == D_ && R == R_) {                                                              \
        launch_attention_pair<D_, R_>(s, cus, k, decoder, a.f32_cache, splits, a.kv_heads, a.heads, a.batch); \
        return hipGetLastError();                                                                   \
    }

hipError_t launch_decode_attention_q8(hipStream_t s, int cus, const AttentionArgs &a, void *scratch,
                                      size_t scratch_bytes) {
    const bool decoder = a.q_norm != nullptr;
    const uint32_t R = a.heads / a.kv_heads;
    if (!attention_supported(a.head_dim, R)) {
        // The entry points' other shapes: the one-workgroup-per-head kernel
        // (no records, no merge).
        if (decoder || a.prefill || !attention_generic_supported(a.head_dim) ||
            (!a.f32_cache && a.head_dim % 64 != 0) || a.batch > 65535)
            return hipErrorNotSupported;
        AttnKernelArgs g{};
        g.query = a.query;
        g.query_stride = a.query_stride ? a.query_stride : a.heads * a.head_dim;
        g.k_scales = a.k_scales;
        g.k_codes = a.k_codes;
        g.v_scales = a.v_scales;
        g.v_codes = a.v_codes;
        g.cached = a.cached;
        g.heads = a.heads;
        g.kv_heads = a.kv_heads;
        g.scale_stride = a.scale_stride;
        g.code_stride = a.code_stride;
        g.scaling = kLog2e / sqrtf((float)a.head_dim);  // kernels.zig:727, in base 2
        g.out = a.out;
        const dim3 grid(a.heads, a.batch);
        if (a.f32_cache) attention_generic_kernel<true><<<grid, 256, 0, s>>>(g, a.head_dim);
        else attention_generic_kernel<false><<<grid, 256, 0, s>>>(g, a.head_dim);
        return hipGetLastError();
    }
    uint32_t chunk, splits;
    plan::attention_shape(cus, a, decoder, chunk, splits);
    // Every range writes a record: refuse a scratch that cannot hold them.
    if (plan::record_bytes(a, splits) > scratch_bytes) return hipErrorInvalidValue;
    AttnKernelArgs k{};
    k.query = a.query;
    k.query_stride = a.query_stride ? a.query_stride : a.heads * a.head_dim;
    if (a.query_slices > kMaxQuerySlices) return hipErrorInvalidValue;
    k.query_slices = a.query_slices;
    k.query_plane = a.query_plane;
    if (a.prefill && !decoder) return hipErrorInvalidValue;
    k.attend_newest = a.prefill ? 1u : 0u;
    k.k_scales = a.k_scales;
    k.k_codes = a.k_codes;
    k.v_scales = a.v_scales;
    k.v_codes = a.v_codes;
    k.cached_dev = a.cached_dev;
    k.cached = a.cached;
    k.cached_bias = a.cached_bias;
    k.rows = a.capacity;
    k.heads = a.heads;
    k.kv_heads = a.kv_heads;
    k.chunk = chunk;
    k.splits = splits;
    k.scale_stride = a.scale_stride;
    k.code_stride = a.code_stride;
    k.scaling = kLog2e / sqrtf((float)a.head_dim);  // kernels.zig:727, in base 2
    k.partial = static_cast<float *>(scratch);
    k.out = a.out;
    k.q_norm = a.q_norm;
    k.k_norm = a.k_norm;
    k.rope_now = a.rope_now;
    k.eps = a.eps;
    if (a.digits) {
        const uint32_t tiles = (a.batch + 15) / 16;
        k.digits = static_cast<uint8_t *>(a.digits);
        k.digit_mult = reinterpret_cast<float *>(k.digits + (size_t)tiles * (a.heads * a.head_dim / 64) * 3 * 16 * 64);
    }
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

hipError_t launch_prefill_append(hipStream_t s, const AttentionArgs &a, uint32_t first, uint32_t count) {
    if (count == 0) return hipSuccess;
    if (!a.k_norm || !a.rope_now || count > 65535 || a.query_slices > kMaxQuerySlices) return hipErrorInvalidValue;
    AttnKernelArgs k{};
    k.query = a.query;
    k.query_stride = a.query_stride;
    k.query_slices = a.query_slices;
    k.query_plane = a.query_plane;
    k.k_scales = a.k_scales;
    k.k_codes = a.k_codes;
    k.v_scales = a.v_scales;
    k.v_codes = a.v_codes;
    k.heads = a.heads;
    k.kv_heads = a.kv_heads;
    k.k_norm = a.k_norm;
    k.rope_now = a.rope_now;
    k.eps = a.eps;
    const dim3 grid(a.kv_heads, count);
#define QWH_APPEND_CASE(D_)                                                                   \
    if (a.head_dim == D_) {                                                                   \
        if (a.f32_cache) prefill_append_kernel<D_, true><<<grid, D_, 0, s>>>(k, first);      \
        else prefill_append_kernel<D_, false><<<grid, D_, 0, s>>>(k, first);                 \
        return hipGetLastError();                                                             \
    }
    QWH_APPEND_CASE(64)
    QWH_APPEND_CASE(128)
    QWH_APPEND_CASE(256)
#undef QWH_APPEND_CASE
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
