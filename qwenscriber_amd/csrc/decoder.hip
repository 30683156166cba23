// The decoder step of decoder.zig:133-339 (forwardToken / step /
// argmaxLogits) for `batch` independent sequences, with its glue kernels.
//
// Everything a step depends on lives on the device: the tokens, each
// sequence's position, the caches and all scratch. A step therefore captures
// once into a HIP graph and replays without host work; a greedy loop replays
// it back to back, the argmax of one step feeding the embedding of the next.
//
// Per layer (decoder.zig:164-272), at batch 1:
//   gemv q4     rmsNormInto(attention_norm) formed in the GEMV prologue;
//               q | k | v rows fused into one matrix
//   attention   per-head rmsNorm of q and k, ropeInPlace at the position,
//               appendCacheRow (q8) of k and v, decodeAttentionStepQ8 over
//               position + 1 rows (split over position ranges)
//   combine     merge of the ranges
//   gemv q4     out projection, residual added in the GEMV epilogue
//   gemv q4     rmsNormInto(ffn_norm) in the prologue; gate and up rows
//               interleaved, siluMul of each pair in the epilogue
//   gemv q4     down projection, residual added
// then rmsNormInto(final) + lm_head GEMV -> argmax (first maximum wins).
// At batch > 1 each GEMV is a digit-plane pass plus the matrix-core GEMV.
// Shapes without a fused GEMV kernel (or QWH_DECODER_UNFUSED set) run the
// norm / digit-plane kernels below as separate launches instead.
//
// Every matrix keeps the format it was bound in (kernels.zig:182-206 applies
// whatever storage a Matrix holds): q4 runs the hex-digit GEMV, q5 and q8 the
// byte-plane GEMV (batch 1 and the per-token path), f32 and f16 the dense
// GEMV (every batch), and at batch > 1 q4, q5 and q8 share the matrix-core
// GEMV when every matrix has that form. The key/value cache is q8 or f32
// (model_config.zig:44-68 CacheFormat; decoder.zig:68-106, :220-253).
#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstring>
#include <vector>

#include "common.h"
#include "device.h"

namespace qwh {
namespace {

// Synthetic model stream ids: identical to the CPU oracle's (the synthetic
// model specification shared by both sides).
constexpr uint32_t kStreamEmbed = 1;
constexpr uint32_t kStreamLmHead = 2;
constexpr uint32_t kStreamLayerBase = 16;    // + 16 * layer + {0 q,1 k,2 v,3 o,4 gate,5 up,6 down}
constexpr uint32_t kStreamCacheBase = 0x10000; // + 0x100 * seq + 2 * layer + {0 keys, 1 values}

// Writes this thread's 8 activations as digit-plane column q of chunk
// `chunk`. The 4 threads of a chunk are consecutive lanes and all call this.
__device__ __forceinline__ void emit_digits(const float v[8], bool valid, size_t chunk, uint32_t q,
                                            uint32_t *words, float *mult) {
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) amax = fmaxf(amax, fabsf(v[k]));
    amax = fmaxf(amax, dev::xor_lane<1>(amax));
    amax = fmaxf(amax, dev::xor_lane<2>(amax));
    const int e = dev::chunk_exponent(amax);
    uint32_t planes[6];
    dev::encode_digits8(v, e, planes);
    if (valid) {
        uint32_t *dst = words + chunk * dev::kChunkWords + q;
#pragma unroll
        for (int j = 0; j < 6; ++j) dst[j * 4] = planes[j];
        if (q == 0) mult[chunk] = __builtin_ldexpf(1.0f, e - 22);
    }
}

// Deterministic block sum (256 threads): wave sums, then the four wave totals
// in order.
__device__ __forceinline__ float block_sum256(float v, float *lds) {
    v = dev::wave_sum(v);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) lds[wave] = v;
    __syncthreads();
    const float total = ((lds[0] + lds[1]) + lds[2]) + lds[3];
    __syncthreads();
    return total;
}

// decoder.zig:346-376 embeddingRow of one token: f32 rows copied, f16 rows
// widened, quantized rows dequantized (quant.zig:315-345 dequantizeGroup in
// the matrix's format: f32(u - bias) times the group's scale); the
// workgroup's threads stride over the row.
__device__ __forceinline__ void embed_row(uint32_t token, int32_t format, const uint16_t *scales, const uint8_t *data,
                                          uint32_t cols, float *out) {
    if (format == QWH_FORMAT_F32) {  // decoder.zig:349-353: the row as it is
        const float *row = reinterpret_cast<const float *>(data) + (size_t)token * cols;
        for (uint32_t i = threadIdx.x; i < cols; i += blockDim.x) out[i] = row[i];
        return;
    }
    if (format == QWH_FORMAT_F16) {  // :354-360: each value widened (fromF16)
        const uint16_t *row = reinterpret_cast<const uint16_t *>(data) + (size_t)token * cols;
        for (uint32_t i = threadIdx.x; i < cols; i += blockDim.x) out[i] = dev::f16_bits_to_f32(row[i]);
        return;
    }
    const uint32_t gpr = cols / 64;
    const uint16_t *row_scales = scales + (size_t)token * gpr;
    if (format == QWH_FORMAT_Q4) {
        const uint8_t *row = data + (size_t)token * (cols / 2);
        for (uint32_t i = threadIdx.x; i < cols / 2; i += blockDim.x) {
            const uint32_t byte = row[i];
            const float s = dev::f16_bits_to_f32(row_scales[(2 * i) / 64]);
            out[2 * i] = __fmul_rn((float)((int)(byte & 0xfu) - 8), s);
            out[2 * i + 1] = __fmul_rn((float)((int)(byte >> 4) - 8), s);
        }
    } else if (format == QWH_FORMAT_Q8) {
        const uint8_t *row = data + (size_t)token * cols;
        for (uint32_t i = threadIdx.x; i < cols; i += blockDim.x)
            out[i] = __fmul_rn((float)((int)row[i] - 128), dev::f16_bits_to_f32(row_scales[i / 64]));
    } else {
        // q5: low nibble as q4, fifth bit j % 8 of byte 32 + j / 8 of the group.
        const uint8_t *row = data + (size_t)token * gpr * 40;
        for (uint32_t i = threadIdx.x; i < cols; i += blockDim.x) {
            const uint8_t *g = row + (size_t)(i / 64) * 40;
            const uint32_t j = i % 64;
            const uint32_t low = (g[j / 2] >> (4 * (j & 1))) & 0xfu;
            const uint32_t high = (g[32 + j / 8] >> (j % 8)) & 1u;
            out[i] = __fmul_rn((float)((int)(low | (high << 4)) - 16), dev::f16_bits_to_f32(row_scales[i / 64]));
        }
    }
}

// The step's embedding: embed_row of each sequence's token; or, for a
// sequence whose row flag is set, decoder.zig:144-147: the given audio row
// replaces the embedding. Also copies the RoPE table row of the sequence's
// position (cos then sin, 2 * half values) to rope_now, so the step's
// attention kernels read it without first waiting for the position.
__global__ __launch_bounds__(256) void embed_kernel(const uint32_t *tokens, int32_t format, const uint16_t *scales,
                                                    const uint8_t *data, uint32_t cols, float *hidden,
                                                    const uint32_t *pos, const float *rope_cos,
                                                    const float *rope_sin, uint32_t half, float *rope_now,
                                                    const float *rows, const uint32_t *row_flags) {
    const uint32_t b = blockIdx.x;
    if (threadIdx.x < 2 * half) {
        const uint32_t p = pos[b];
        const uint32_t t = threadIdx.x;
        rope_now[(size_t)b * 2 * half + t] = t < half ? rope_cos[(size_t)p * half + t] : rope_sin[(size_t)p * half + t - half];
    }
    float *out = hidden + (size_t)b * cols;
    if (row_flags[b]) {
        const float *src = rows + (size_t)b * cols;
        for (uint32_t i = threadIdx.x; i < cols; i += blockDim.x) out[i] = src[i];
        return;
    }
    embed_row(tokens[b], format, scales, data, cols, out);
}

// The prompt rows of a prefill (decoder.zig:308-333): row i is the embedding
// of tokens[i], or, where row_index[i] is not ~0u, that row of the projected
// audio features; rope_rows[i] gets the RoPE table row of position first + i.
__global__ __launch_bounds__(256) void embed_prompt_kernel(const uint32_t *tokens, const uint32_t *row_index,
                                                           int32_t format, const uint16_t *scales,
                                                           const uint8_t *data, uint32_t cols, float *hidden,
                                                           uint32_t first, const float *rope_cos,
                                                           const float *rope_sin, uint32_t half, float *rope_rows,
                                                           const float *audio_rows) {
    const uint32_t i = blockIdx.x;
    if (threadIdx.x < 2 * half) {
        const uint32_t p = first + i;
        const uint32_t t = threadIdx.x;
        rope_rows[(size_t)i * 2 * half + t] = t < half ? rope_cos[(size_t)p * half + t] : rope_sin[(size_t)p * half + t - half];
    }
    float *out = hidden + (size_t)i * cols;
    if (row_index[i] != ~0u) {
        const float *src = audio_rows + (size_t)row_index[i] * cols;
        for (uint32_t c = threadIdx.x; c < cols; c += blockDim.x) out[c] = src[c];
        return;
    }
    embed_row(tokens[i], format, scales, data, cols, out);
}

// kernels.zig:274-300 rmsNormInto + math.zig:120-130, emitting the
// normalized row as digit planes for the next GEMV. One block per sequence.
__global__ __launch_bounds__(256) void rmsnorm_digits_kernel(const float *x, const float *weight,
                                                             uint32_t cols, float eps, uint32_t *words,
                                                             float *mult) {
    __shared__ float lds[4];
    const uint32_t b = blockIdx.x;
    const float *row = x + (size_t)b * cols;
    const uint32_t groups8 = cols / 8;
    const uint32_t iters = (groups8 + 255) / 256;
    float ss = 0.0f;
    for (uint32_t it = 0; it < iters; ++it) {
        const uint32_t g8 = threadIdx.x + it * 256;
        if (g8 < groups8) {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const float v = row[g8 * 8 + k];
                ss = __fadd_rn(ss, __fmul_rn(v, v));
            }
        }
    }
    const float sum_squares = block_sum256(ss, lds);
    const float mean_square = __fdiv_rn(sum_squares, (float)cols);
    const float inverse_rms = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(mean_square, eps)));
    const uint32_t T = cols / 32;
    for (uint32_t it = 0; it < iters; ++it) {
        const uint32_t g8 = threadIdx.x + it * 256;
        const bool valid = g8 < groups8;
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k)
            v[k] = valid ? __fmul_rn(__fmul_rn(row[g8 * 8 + k], inverse_rms), weight[g8 * 8 + k]) : 0.0f;
        emit_digits(v, valid, (size_t)b * T + g8 / 4, g8 & 3u, words, mult);
    }
}

// argmaxLogits (decoder.zig:290-301): the largest value, the lowest index
// among equal maxima. Stage 1: one partial per block of kArgmaxPerBlock
// logits, four consecutive logits per thread (one 16-byte load where the
// block's logits start 16-byte aligned), merged across the wavefront and
// then the workgroup.
// The merge order does not matter: `better` picks the same (value, index)
// from any order, and never takes a NaN.
constexpr uint32_t kArgmaxPerBlock = 1024;

__device__ __forceinline__ void better(float &v, uint32_t &i, float v2, uint32_t i2) {
    if (v2 > v || (v2 == v && i2 < i)) {
        v = v2;
        i = i2;
    }
}

__device__ __forceinline__ void wave_better(float &v, uint32_t &i) {
#pragma unroll
    for (int mask = 32; mask >= 1; mask >>= 1) {
        const float v2 = __shfl_xor(v, mask, 64);
        const uint32_t i2 = __shfl_xor(i, mask, 64);
        better(v, i, v2, i2);
    }
}

__global__ __launch_bounds__(256) void argmax_partial_kernel(const float *logits, uint32_t count,
                                                             uint32_t per_block, float *pv, uint32_t *pi) {
    const uint32_t b = blockIdx.y;
    const float *row = logits + (size_t)b * count;
    const uint32_t start = blockIdx.x * per_block;
    const uint32_t end = min(start + per_block, count);
    // 16-byte loads where the block's first logit is 16-byte aligned (every
    // later load of the thread then is too: the stride is 4 KiB).
    const bool aligned = (reinterpret_cast<uintptr_t>(row + start) & 15u) == 0;
    float bv = -FLT_MAX;
    uint32_t bi = 0xffffffffu;
    for (uint32_t i = start + threadIdx.x * 4; i < end; i += blockDim.x * 4) {
        if (aligned && i + 4 <= end) {
            const float4 v = *reinterpret_cast<const float4 *>(row + i);
            better(bv, bi, v.x, i);
            better(bv, bi, v.y, i + 1);
            better(bv, bi, v.z, i + 2);
            better(bv, bi, v.w, i + 3);
        } else {
            for (uint32_t e = i; e < i + 4 && e < end; ++e) better(bv, bi, row[e], e);
        }
    }
    wave_better(bv, bi);
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
    const uint32_t wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sv[wave] = bv;
        si[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t w = 1; w < blockDim.x / 64; ++w) better(bv, bi, sv[w], si[w]);
        // A NaN first logit stays the reference's best (no value compares
        // greater than it): index 0 then wins outright.
        const bool nan_first = blockIdx.x == 0 && row[0] != row[0];
        pv[(size_t)b * gridDim.x + blockIdx.x] = nan_first ? INFINITY : bv;
        pi[(size_t)b * gridDim.x + blockIdx.x] = nan_first ? 0u : bi;
    }
}

// The best of row b's `parts` partials, by a 256-thread workgroup: four
// partials per thread requested together, merged over the wavefront and
// then the four wavefronts; the result is valid in thread 0.
__device__ __forceinline__ void best_of_partials(const float *pv, const uint32_t *pi, uint32_t parts, uint32_t b,
                                                 float &bv, uint32_t &bi) {
    bv = -FLT_MAX;
    bi = 0xffffffffu;
    const float *rv = pv + (size_t)b * parts;
    const uint32_t *ri = pi + (size_t)b * parts;
    for (uint32_t p0 = 0; p0 < parts; p0 += 1024) {
        float v[4];
        uint32_t idx[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t p = p0 + threadIdx.x + 256 * q;
            const uint32_t pc = p < parts ? p : parts - 1;
            v[q] = rv[pc];
            idx[q] = ri[pc];
        }
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (p0 + threadIdx.x + 256 * q < parts) better(bv, bi, v[q], idx[q]);
    }
    wave_better(bv, bi);
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = bv;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0)
        for (int w = 1; w < 4; ++w) better(bv, bi, sv[w], si[w]);
}

// argmaxLogits of each row from the partials: ids[b].
__global__ __launch_bounds__(256) void argmax_rows_finish_kernel(const float *pv, const uint32_t *pi, uint32_t parts,
                                                                 uint32_t *ids) {
    const uint32_t b = blockIdx.x;
    float bv;
    uint32_t bi;
    best_of_partials(pv, pi, parts, b, bv, bi);
    // A row with no value above -FLT_MAX (all -inf or NaN) is the
    // reference's index 0.
    if (threadIdx.x == 0) ids[b] = bi == 0xffffffffu ? 0u : bi;
}

// Greedy generation with stop rules (wasm/model.zig:423-451 decodeStep,
// :495-499 endsSequence), per sequence, in device memory: `mode` 0 = plain
// steps; 1 = stop on a stop token or the token budget. done[b] freezes a
// finished sequence (its position, token and history no longer change);
// count[b] is the number of ids it has emitted into history rows.
struct GenState {
    uint32_t mode;
    uint32_t budget;
    uint32_t stops[3];
    uint32_t stop_count;
    uint32_t pad[2];
    // then done[batch], count[batch]
};

__device__ __forceinline__ bool is_stop(const GenState *g, uint32_t token) {
    for (uint32_t i = 0; i < g->stop_count && i < 3; ++i)
        if (token == g->stops[i]) return true;
    return false;
}

// Stage 2: merges the partials and writes the next token. Plain steps record
// it in the history at (position - history base) and advance the position.
// With stop rules (decodeStep): the forward that produced the token has run,
// so the position advances; a stop token ends the sequence without being
// emitted; otherwise it is emitted at row count[b], and the sequence ends
// once it has emitted `budget` ids. A finished sequence is left unchanged
// (its step recomputes the same row and writes nothing).
__global__ __launch_bounds__(256) void argmax_finish_kernel(const float *pv, const uint32_t *pi,
                                                            uint32_t parts, uint32_t *tokens, uint32_t *pos,
                                                            const uint32_t *hist_base, uint32_t *history,
                                                            uint32_t batch, uint32_t history_rows,
                                                            const GenState *gen, uint32_t *done, uint32_t *count) {
    const uint32_t b = blockIdx.x;
    float bv;
    uint32_t bi;
    best_of_partials(pv, pi, parts, b, bv, bi);
    if (threadIdx.x == 0) {
        // A row of NaN logits leaves no index; the reference then returns 0.
        const uint32_t token = bi == 0xffffffffu ? 0u : bi;
        const uint32_t p = pos[b];
        if (gen->mode == 1) {
            if (done[b]) return;
            pos[b] = p + 1;
            tokens[b] = token;
            if (is_stop(gen, token)) {
                done[b] = 1;
                return;
            }
            const uint32_t n = count[b];
            if (n < history_rows) history[(size_t)n * batch + b] = token;
            count[b] = n + 1;
            if (n + 1 >= gen->budget) done[b] = 1;
            return;
        }
        tokens[b] = token;
        if (history) {
            const uint32_t row = p - hist_base[b];
            if (row < history_rows) history[(size_t)row * batch + b] = token;
        }
        pos[b] = p + 1;
    }
}

__global__ void advance_kernel(uint32_t *pos, uint32_t batch) {
    const uint32_t b = threadIdx.x;
    if (b < batch) pos[b] += 1;
}

__global__ void fill_kernel(float *dst, uint64_t count, float value) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) dst[i] = value;
}

}  // namespace
}  // namespace qwh

using qwh::Matrix;

struct qwh_decoder {
    qwh_ctx *ctx = nullptr;
    qwh_decoder_config c{};
    uint32_t batch = 0;
    uint32_t qw = 0, kvw = 0;
    struct Layer {
        Matrix qkv, o, gu, down;
        float *attn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr, *ffn_norm = nullptr;
    };
    std::vector<Layer> layers;
    Matrix embed, lm_head;
    float *final_norm = nullptr;
    float *rope_cos = nullptr, *rope_sin = nullptr;
    float *rope_now = nullptr;  // per sequence: the table row of its current position
    uint8_t *keys = nullptr, *values = nullptr;
    size_t cache_scales = 0, cache_codes = 0, layer_stride = 0, seq_stride = 0;
    uint32_t *tokens_dev = nullptr, *pos_dev = nullptr, *hist_base_dev = nullptr, *history_dev = nullptr;
    uint32_t history_rows = 0;
    float *hidden = nullptr, *qkv = nullptr, *attn = nullptr, *gu = nullptr, *logits = nullptr;
    void *digits = nullptr;
    void *attn_scratch = nullptr;
    size_t attn_scratch_bytes = 0;
    float *arg_v = nullptr;
    uint32_t *arg_i = nullptr;
    uint32_t arg_parts = 0, arg_per_block = 0;
    uint32_t *host_stage = nullptr;  // pinned: tokens in / ids out, then the row flags, then generation state
    float *rows_dev = nullptr;        // audio rows for the next forward_rows step
    uint32_t *row_flags_dev = nullptr;  // per sequence: 1 = take rows_dev's row, not the embedding
    std::vector<uint32_t> pos_host;
    std::vector<void *> allocations;
    hipGraphExec_t graph[2] = {nullptr, nullptr};
    bool use_graph = true;
    int32_t cache_format = QWH_CACHE_Q8;
    // Generation state (GenState, then done[batch], count[batch]) and the
    // mode last written to it.
    void *gen = nullptr;
    uint32_t gen_mode = 0;
    // The step's kernel plan, decided from the bound matrices' formats before
    // the step is first enqueued (and again after a matrix changes format).
    bool planned = false;
    bool fused = true;  // every q4 GEMV forms its own activations (no norm / prep kernels)
    bool batched = false;  // batch > 1: int8 digit planes + matrix-core GEMV
    // Per-token q4 GEMVs (fused, not batched): the embedding gathered by the
    // first q | k | v GEMV, the argmax partials formed by the lm_head GEMV.
    bool fold_embed = false, fold_argmax = false;
    void *batch_digits = nullptr;
    // Batched: K-slice partial sums. When every layer matrix has a split
    // form (split_parts), the o, gate|up and down GEMVs leave their partial
    // sums here and the prep that follows adds them (q|k|v reduces its own).
    float *parts = nullptr;
    bool split_parts = false;
    uint32_t slices_o = 0, slices_gu = 0, slices_down = 0, slices_qkv = 0;
    // qwh_decoder_prefill's buffers, for up to kPrefillChunk prompt positions
    // of one sequence, allocated at its first call.
    struct PrefillBuffers {
        float *hidden = nullptr, *qkv = nullptr, *attn = nullptr, *rope = nullptr, *parts = nullptr;
        float *wide = nullptr;  // the rows form's siluMul(gate, up) rows
        void *digits = nullptr, *attn_scratch = nullptr, *arg_scratch = nullptr;
        size_t attn_scratch_bytes = 0;
        uint32_t *staged_dev = nullptr;  // tokens, audio row indices, positions
        uint32_t *id_dev = nullptr;
        uint32_t *host = nullptr;        // pinned: the same three arrays, then the id
    } pf;
};

namespace qwh {
namespace {

int32_t dalloc(qwh_decoder *d, size_t bytes, void **out) {
    void *p = nullptr;
    const hipError_t err = hipMalloc(&p, bytes ? bytes : 1);
    if (err != hipSuccess) {
        (void)hipGetLastError();
        return fail(d->ctx, QWH_E_OUT_OF_MEMORY, "hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(err));
    }
    // Zeroed once here (at set-up, outside any graph), so that no buffer
    // starts with stale bits: e.g. the digit planes of token slots past the
    // batch, which some writers leave alone. On the context's stream, which
    // does not wait for the default stream: the writes that follow on it
    // must come after the zeros.
    const hipError_t zero = hipMemsetAsync(p, 0, bytes ? bytes : 1, d->ctx->stream);
    if (zero != hipSuccess) {
        (void)hipFree(p);
        return fail(d->ctx, QWH_E_DEVICE, "hipMemset(%zu) failed: %s", bytes, hipGetErrorString(zero));
    }
    d->allocations.push_back(p);
    *out = p;
    return QWH_OK;
}

int32_t alloc_matrix(qwh_decoder *d, Matrix &m, uint32_t rows, uint32_t cols, int32_t format = QWH_FORMAT_Q4) {
    m.format = format;
    m.rows = rows;
    m.cols = cols;
    m.owned = false;  // freed with the decoder's allocations
    if (is_dense_format(format)) {
        m.scales = nullptr;
        return dalloc(d, (size_t)rows * cols * dense_element_bytes(format), reinterpret_cast<void **>(&m.data));
    }
    const size_t groups = (size_t)rows * (cols / 64);
    QWH_TRY(dalloc(d, groups * 2, reinterpret_cast<void **>(&m.scales)));
    QWH_TRY(dalloc(d, groups * (size_t)data_bytes_per_group(format), reinterpret_cast<void **>(&m.data)));
    return QWH_OK;
}

void dfree(qwh_decoder *d, void *p) {
    if (!p) return;
    auto it = std::find(d->allocations.begin(), d->allocations.end(), p);
    if (it != d->allocations.end()) d->allocations.erase(it);
    (void)hipFree(p);
}

// Captured graphs hold the kernels' arguments (matrix planes among them):
// dropped whenever a matrix moves, and the step planned again.
void invalidate_step(qwh_decoder *d) {
    for (hipGraphExec_t &g : d->graph)
        if (g) {
            (void)hipGraphExecDestroy(g);
            g = nullptr;
        }
    d->planned = false;
}

// Re-creates a decoder matrix (zeroed) in `format` when it holds another:
// the planes of a fused block (q | k | v, gate | up) share one format, so a
// member bound in a new format re-creates the whole block and the other
// members are bound again after it.
int32_t ensure_format(qwh_decoder *d, Matrix &m, int32_t format) {
    if (m.format == format) return QWH_OK;
    QWH_TRY(check_hip(d->ctx, hipStreamSynchronize(d->ctx->stream), "matrix format change"));
    invalidate_step(d);
    dfree(d, m.scales);
    dfree(d, m.data);
    m.scales = m.data = nullptr;
    return alloc_matrix(d, m, m.rows, m.cols, format);
}

int32_t fill_ones(qwh_decoder *d, float *dst, uint64_t count) {
    fill_kernel<<<(unsigned)((count + 255) / 256 < 1024 ? (count + 255) / 256 : 1024), 256, 0, d->ctx->stream>>>(
        dst, count, 1.0f);
    return check_hip(d->ctx, hipGetLastError(), "fill");
}

// The step's kernels for the formats the matrices hold now: q5 / q8
// matrices need the byte-plane GEMV's shapes; the matrix-core batch GEMV
// runs when every matrix has that form (q4, q8), the split form with partial
// sums when o, gate | up and down all split along K.
int32_t plan_step(qwh_decoder *d) {
    const qwh_decoder_config &c = d->c;
    std::vector<const Matrix *> all;
    for (const qwh_decoder::Layer &L : d->layers)
        for (const Matrix *m : {&L.qkv, &L.o, &L.gu, &L.down}) all.push_back(m);
    all.push_back(&d->lm_head);
    bool q4_fused = getenv("QWH_DECODER_UNFUSED") == nullptr;
    bool batch_form = d->batch > 1 && getenv("QWH_DECODER_PER_TOKEN") == nullptr;
    for (const Matrix *m : all) {
        if (m->format == QWH_FORMAT_Q4) {
            q4_fused = q4_fused && gemv_q4_fused_supported(m->rows, m->cols);
        } else if (is_dense_format(m->format)) {
            if (!gemv_dense_supported(m->format, m->cols))
                return fail(d->ctx, QWH_E_UNSUPPORTED, "no GEMV for a %ux%u matrix of format %d", m->rows, m->cols,
                            m->format);
        } else if (!gemv_b8_supported(m->format, m->rows, m->cols)) {
            return fail(d->ctx, QWH_E_UNSUPPORTED, "no GEMV for a %ux%u matrix of format %d", m->rows, m->cols,
                        m->format);
        }
        batch_form = batch_form && gemv_batch_supported(*m);
    }
    d->fused = q4_fused;
    d->batched = batch_form;
    const bool per_token_q4 = q4_fused && !batch_form;
    const qwh_decoder::Layer &first = d->layers[0];
    d->fold_embed = per_token_q4 && first.qkv.format == QWH_FORMAT_Q4 &&
                    gemv_q4_source_supported(GemvInput::Embed, first.qkv.rows, first.qkv.cols);
    d->fold_argmax = per_token_q4 && d->lm_head.format == QWH_FORMAT_Q4;
    d->split_parts = false;
    d->slices_o = d->slices_gu = d->slices_down = d->slices_qkv = 0;
    if (d->batched) {
        const qwh_decoder::Layer &L0 = d->layers[0];
        d->slices_qkv = batch_slices(L0.qkv);
        d->slices_o = batch_slices(L0.o);
        d->slices_gu = batch_slices(L0.gu);
        d->slices_down = batch_slices(L0.down);
        d->split_parts = d->slices_o && d->slices_gu && d->slices_down && d->parts &&
                         getenv("QWH_DECODER_NO_SPLIT") == nullptr;
    }
    (void)c;
    d->planned = true;
    return QWH_OK;
}

// Enqueues one decoder step for every sequence (tokens and positions read
// from device memory).
int32_t enqueue_step(qwh_decoder *d, bool want_logits) {
    qwh_ctx *ctx = d->ctx;
    hipStream_t s = ctx->stream;
    const qwh_decoder_config &c = d->c;
    const uint32_t B = d->batch;
    uint32_t *words = static_cast<uint32_t *>(d->digits);
    auto mult_of = [&](uint32_t cols) {
        return reinterpret_cast<float *>(words + (size_t)B * (cols / 32) * dev::kChunkWords);
    };
    hipError_t err = hipSuccess;
    // W * f(x) for one of the decoder's activation forms: in one kernel when
    // the GEMV forms them itself, else through a digit-plane pass.
    // Batched with split_parts: the partial sums the next prep adds (the
    // residual stream's pending update, or the gate / up pairs).
    PartialSums pending;
    auto gemv = [&](GemvInput::Mode mode, const float *x, const float *norm, const Matrix &w, float *out,
                    const float *residual, bool pairs) -> hipError_t {
        GemvInput in;
        in.mode = mode;
        in.x = x;
        in.norm = norm;
        in.eps = c.eps;
        in.pairs = pairs;
        if (d->batched) {
            if (mode != GemvInput::Digits) {  // Digits: the planes are already in batch_digits
                const hipError_t e = launch_prep_batch(s, in, B, w.cols, d->batch_digits, &pending);
                pending = PartialSums{};
                if (e != hipSuccess) return e;
            }
            BatchNorm bn;
            bn.rms = mode == GemvInput::RmsNorm;
            bn.eps = c.eps;
            return launch_gemv_batch(s, d->batch_digits, w, B, out, residual, pairs, d->parts, bn);
        }
        if (is_dense_format(w.format)) return launch_gemv_dense(s, ctx->cus, in, w, B, out, residual);
        if (w.format != QWH_FORMAT_Q4) return launch_gemv_b8(s, ctx->cus, in, w, B, out, residual);
        if (d->fused) return launch_gemv_q4_src(s, ctx->cus, in, w, B, out, residual);
        if (mode == GemvInput::RmsNorm) {
            rmsnorm_digits_kernel<<<B, 256, 0, s>>>(x, norm, w.cols, c.eps, words, mult_of(w.cols));
        } else {
            const hipError_t e = launch_prep_q4(s, x, B, w.cols, words);
            if (e != hipSuccess) return e;
        }
        GemvInput pre;
        pre.mode = GemvInput::Digits;
        pre.digits = words;
        pre.pairs = pairs;
        return launch_gemv_q4_src(s, ctx->cus, pre, w, B, out, residual);
    };
    if (!d->fold_embed)
        embed_kernel<<<B, 256, 0, s>>>(d->tokens_dev, d->embed.format,
                                       reinterpret_cast<const uint16_t *>(d->embed.scales), d->embed.data, c.hidden,
                                       d->hidden, d->pos_dev, d->rope_cos, d->rope_sin, c.head_dim / 2, d->rope_now,
                                       d->rows_dev, d->row_flags_dev);
    for (uint32_t l = 0; l < c.layers && err == hipSuccess; ++l) {
        qwh_decoder::Layer &L = d->layers[l];
        // Batched with a K split: q | k | v stay partial sums, added by the
        // attention kernels as they read them (no reduce launch).
        const bool qkv_parts = d->batched && d->slices_qkv > 1 && d->parts;
        if (qkv_parts) {
            GemvInput in;
            in.mode = GemvInput::RmsNorm;
            in.x = d->hidden;
            in.norm = L.attn_norm;
            in.eps = c.eps;
            err = launch_prep_batch(s, in, B, c.hidden, d->batch_digits, &pending);
            pending = PartialSums{};
            if (err != hipSuccess) break;
            BatchNorm bn;
            bn.rms = true;
            bn.eps = c.eps;
            err = launch_gemv_batch_parts(s, d->batch_digits, L.qkv, B, d->parts, bn);
        } else if (l == 0 && d->fold_embed) {
            // embeddingRow (or the audio row) formed by every workgroup; the
            // first stores it to the residual stream, with the RoPE row.
            GemvInput in;
            in.mode = GemvInput::Embed;
            in.norm = L.attn_norm;
            in.eps = c.eps;
            in.tokens = d->tokens_dev;
            in.embed = &d->embed;
            in.rows = d->rows_dev;
            in.row_flags = d->row_flags_dev;
            in.embed_out = d->hidden;
            in.pos = d->pos_dev;
            in.rope_cos = d->rope_cos;
            in.rope_sin = d->rope_sin;
            in.rope_half = c.head_dim / 2;
            in.rope_now = d->rope_now;
            err = launch_gemv_q4_src(s, ctx->cus, in, L.qkv, B, d->qkv, nullptr);
        } else {
            err = gemv(GemvInput::RmsNorm, d->hidden, L.attn_norm, L.qkv, d->qkv, nullptr, false);
        }
        if (err != hipSuccess) break;
        // Per-head norms, RoPE, the cache append and the attention itself
        // (decoder.zig:180-253) in one launch.
        uint8_t *kl = d->keys + (size_t)l * d->layer_stride;
        uint8_t *vl = d->values + (size_t)l * d->layer_stride;
        AttentionArgs aa{};
        aa.out = d->attn;
        aa.query = qkv_parts ? d->parts : d->qkv;
        aa.query_stride = d->qw + 2 * d->kvw;
        if (qkv_parts) {
            aa.query_slices = d->slices_qkv;
            aa.query_plane = (uint64_t)B * (d->qw + 2 * d->kvw);
        }
        aa.q_norm = L.q_norm;
        aa.k_norm = L.k_norm;
        aa.rope_now = d->rope_now;
        aa.eps = c.eps;
        aa.k_scales = kl;
        aa.k_codes = kl + d->cache_scales;
        aa.v_scales = vl;
        aa.v_codes = vl + d->cache_scales;
        aa.cached_dev = d->pos_dev;
        aa.cached_bias = 1;
        aa.capacity = c.max_positions;
        aa.heads = c.heads;
        aa.kv_heads = c.kv_heads;
        aa.head_dim = c.head_dim;
        aa.batch = B;
        aa.scale_stride = d->seq_stride;
        aa.code_stride = d->seq_stride;
        aa.f32_cache = d->cache_format == QWH_CACHE_F32;
        // Batched: the attention output also arrives as the O projection's
        // digit planes.
        aa.digits = d->batched ? d->batch_digits : nullptr;
        err = launch_decode_attention_q8(s, ctx->cus, aa, d->attn_scratch, d->attn_scratch_bytes);
        if (err != hipSuccess) break;
        if (d->split_parts) {
            // o, gate|up, down as partial sums; each prep adds the previous
            // one's (hidden += o; siluMul(gate, up); hidden += down at the
            // next layer's or the final prep).
            err = launch_gemv_batch_parts(s, d->batch_digits, L.o, B, d->parts);
            if (err != hipSuccess) break;
            GemvInput norm_in;
            norm_in.mode = GemvInput::RmsNorm;
            norm_in.x = d->hidden;
            norm_in.norm = L.ffn_norm;
            norm_in.eps = c.eps;
            const PartialSums o_sums{d->parts, d->slices_o, c.hidden, false, d->hidden};
            err = launch_prep_batch(s, norm_in, B, c.hidden, d->batch_digits, &o_sums);
            if (err != hipSuccess) break;
            BatchNorm bn;
            bn.rms = true;
            bn.eps = c.eps;
            err = launch_gemv_batch_parts(s, d->batch_digits, L.gu, B, d->parts, bn);
            if (err != hipSuccess) break;
            GemvInput pairs_in;
            pairs_in.mode = GemvInput::F32;
            const PartialSums gu_sums{d->parts, d->slices_gu, 2 * c.ffn, true, nullptr};
            err = launch_prep_batch(s, pairs_in, B, c.ffn, d->batch_digits, &gu_sums);
            if (err != hipSuccess) break;
            err = launch_gemv_batch_parts(s, d->batch_digits, L.down, B, d->parts);
            if (err != hipSuccess) break;
            pending = PartialSums{d->parts, d->slices_down, c.hidden, false, d->hidden};
            continue;
        }
        err = gemv(d->batched ? GemvInput::Digits : GemvInput::F32, d->attn, nullptr, L.o, d->hidden, d->hidden,
                   false);
        if (err != hipSuccess) break;
        // gate | up rows interleaved: the GEMV writes siluMul(gate, up).
        err = gemv(GemvInput::RmsNorm, d->hidden, L.ffn_norm, L.gu, d->gu, nullptr, true);
        if (err != hipSuccess) break;
        err = gemv(GemvInput::F32, d->gu, nullptr, L.down, d->hidden, d->hidden, false);
    }
    if (err == hipSuccess) {
        if (want_logits) {
            uint32_t parts = d->arg_parts;
            if (d->fold_argmax) {
                // The lm_head GEMV leaves a (value, row) partial per workgroup.
                GemvInput in;
                in.mode = GemvInput::RmsNorm;
                in.x = d->hidden;
                in.norm = d->final_norm;
                in.eps = c.eps;
                in.arg_value = d->arg_v;
                in.arg_index = d->arg_i;
                parts = gemv_q4_partials(ctx->cus, d->lm_head, in);
                err = parts && parts <= kGemvMaxPartials
                          ? launch_gemv_q4_src(s, ctx->cus, in, d->lm_head, B, d->logits, nullptr)
                          : hipErrorInvalidValue;
            } else {
                err = gemv(GemvInput::RmsNorm, d->hidden, d->final_norm, d->lm_head, d->logits, nullptr, false);
                if (err == hipSuccess)
                    argmax_partial_kernel<<<dim3(d->arg_parts, B), 256, 0, s>>>(d->logits, c.vocab, d->arg_per_block,
                                                                                 d->arg_v, d->arg_i);
            }
            if (err == hipSuccess) {
                const GenState *gen = static_cast<const GenState *>(d->gen);
                uint32_t *done = reinterpret_cast<uint32_t *>(static_cast<uint8_t *>(d->gen) + sizeof(GenState));
                argmax_finish_kernel<<<B, 256, 0, s>>>(d->arg_v, d->arg_i, parts, d->tokens_dev, d->pos_dev,
                                                       d->hist_base_dev, d->history_dev, B, d->history_rows, gen, done,
                                                       done + B);
                err = hipGetLastError();
            }
        } else {
            advance_kernel<<<1, 64 * ((B + 63) / 64), 0, s>>>(d->pos_dev, B);
            err = hipGetLastError();
        }
    }
    if (err == hipSuccess) err = hipGetLastError();
    return check_hip(ctx, err, "decoder step launch");
}

int32_t run_step(qwh_decoder *d, bool want_logits) {
    qwh_ctx *ctx = d->ctx;
    if (!d->planned) QWH_TRY(plan_step(d));
    if (!d->use_graph) return enqueue_step(d, want_logits);
    hipGraphExec_t &exec = d->graph[want_logits ? 1 : 0];
    if (!exec) {
        QWH_TRY(check_hip(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal), "begin capture"));
        const int32_t st = enqueue_step(d, want_logits);
        hipGraph_t graph = nullptr;
        const hipError_t end = hipStreamEndCapture(ctx->stream, &graph);
        if (st != QWH_OK) {
            if (graph) (void)hipGraphDestroy(graph);
            return st;
        }
        QWH_TRY(check_hip(ctx, end, "end capture"));
        const hipError_t inst = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        QWH_TRY(check_hip(ctx, inst, "graph instantiate"));
    }
    return check_hip(ctx, hipGraphLaunch(exec, ctx->stream), "graph launch");
}

// kernels.zig:534-564 buildRopeTables / inverseFrequency, in f32 on the host
// as model.zig:400-407 does at load time.
void build_rope_tables(std::vector<float> &cos_t, std::vector<float> &sin_t, uint32_t half, float theta,
                       uint32_t max_positions) {
    const uint32_t head_dim = half * 2;
    cos_t.assign((size_t)max_positions * half, 0.0f);
    sin_t.assign((size_t)max_positions * half, 0.0f);
    for (uint32_t p = 0; p < max_positions; ++p) {
        for (uint32_t i = 0; i < half; ++i) {
            const volatile float exponent = -2.0f * (float)i / (float)head_dim;
            const float inv = powf(theta, exponent);
            const volatile float angle = (float)p * inv;
            cos_t[(size_t)p * half + i] = cosf(angle);
            sin_t[(size_t)p * half + i] = sinf(angle);
        }
    }
}

// Copies src's rows to rows row_offset + i * stride of dst (stride 1: a
// contiguous block; stride 2: every other row, for the gate / up pairs).
int32_t copy_rows(qwh_decoder *d, Matrix &dst, uint32_t row_offset, const Matrix &src, uint32_t stride = 1) {
    hipStream_t s = d->ctx->stream;
    if (is_dense_format(dst.format)) {
        const size_t rb = (size_t)dst.cols * dense_element_bytes(dst.format);  // bytes per row
        return check_hip(d->ctx, hipMemcpy2DAsync(dst.data + (size_t)row_offset * rb, rb * stride, src.data, rb, rb,
                                                  src.rows, hipMemcpyDeviceToDevice, s), "copy rows");
    }
    const size_t gpr = dst.cols / 64;
    const size_t sb = gpr * 2, db = gpr * (size_t)data_bytes_per_group(dst.format);  // scale and code bytes per row
    QWH_TRY(check_hip(d->ctx, hipMemcpy2DAsync(dst.scales + (size_t)row_offset * sb, sb * stride, src.scales, sb, sb,
                                               src.rows, hipMemcpyDeviceToDevice, s), "copy scales"));
    QWH_TRY(check_hip(d->ctx, hipMemcpy2DAsync(dst.data + (size_t)row_offset * db, db * stride, src.data, db, db,
                                               src.rows, hipMemcpyDeviceToDevice, s), "copy data"));
    return QWH_OK;
}

// Synthetic values for rows [row_offset, row_offset + rows) of `dst` from
// rows [0, rows) of `stream`, generated in slabs through a temporary f32
// buffer and quantized to dst's format on the device.
int32_t synth_rows(qwh_decoder *d, Matrix &dst, uint32_t row_offset, uint32_t rows, uint32_t seed,
                   uint32_t stream, float scale, float *temp, size_t temp_values) {
    const uint32_t cols = dst.cols;
    const size_t gpr = cols / 64;
    const size_t bpg = (size_t)data_bytes_per_group(dst.format);
    uint32_t slab = (uint32_t)(temp_values / cols);
    if (slab == 0) return fail(d->ctx, QWH_E_INVALID_ARGUMENT, "synthetic slab too small");
    hipStream_t s = d->ctx->stream;
    for (uint32_t r = 0; r < rows; r += slab) {
        const uint32_t n = rows - r < slab ? rows - r : slab;
        const uint64_t count = (uint64_t)n * cols, at = (uint64_t)(row_offset + r) * cols;
        // f32 rows are the values themselves; f16 rows their RNE bits.
        float *values = dst.format == QWH_FORMAT_F32 ? reinterpret_cast<float *>(dst.data) + at : temp;
        QWH_TRY(check_hip(d->ctx, launch_synth_normal(s, seed, stream, (uint64_t)r * cols, count, scale, values),
                          "synthetic values"));
        if (dst.format == QWH_FORMAT_F32) continue;
        if (dst.format == QWH_FORMAT_F16) {
            QWH_TRY(check_hip(d->ctx, launch_f32_to_f16(s, temp, count, reinterpret_cast<uint16_t *>(dst.data) + at),
                              "f16 values"));
            continue;
        }
        QWH_TRY(check_hip(d->ctx, launch_quantize_rows(s, dst.format, temp, (uint64_t)n * gpr,
                                                      dst.scales + (size_t)(row_offset + r) * gpr * 2,
                                                      dst.data + (size_t)(row_offset + r) * gpr * bpg),
                          "quantize"));
    }
    return QWH_OK;
}

int32_t check_matrix(qwh_decoder *d, const Matrix *m, uint32_t rows, uint32_t cols) {
    if (!m) return fail(d->ctx, QWH_E_NOT_FOUND, "unknown matrix handle");
    if (m->format != QWH_FORMAT_Q4 && m->format != QWH_FORMAT_Q5 && m->format != QWH_FORMAT_Q8 &&
        !is_dense_format(m->format))
        return fail(d->ctx, QWH_E_UNSUPPORTED, "decoder matrices are f32, f16, q4, q5 or q8 (formats 0, 1, 16-18), got %d",
                    m->format);
    if (m->rows != rows || m->cols != cols)
        return fail(d->ctx, QWH_E_SHAPE_MISMATCH, "matrix is %ux%u, expected %ux%u", m->rows, m->cols, rows, cols);
    return QWH_OK;
}

}  // namespace
size_t argmax_scratch_bytes(uint32_t rows, uint32_t count) {
    const uint32_t parts = (count + kArgmaxPerBlock - 1) / kArgmaxPerBlock;
    return (size_t)rows * parts * (sizeof(float) + sizeof(uint32_t));
}

hipError_t launch_argmax_rows(hipStream_t s, const float *logits, uint32_t rows, uint32_t count, void *scratch,
                              uint32_t *ids) {
    if (!rows || !count) return hipErrorInvalidValue;
    const uint32_t parts = (count + kArgmaxPerBlock - 1) / kArgmaxPerBlock;
    float *pv = static_cast<float *>(scratch);
    uint32_t *pi = reinterpret_cast<uint32_t *>(pv + (size_t)rows * parts);
    argmax_partial_kernel<<<dim3(parts, rows), 256, 0, s>>>(logits, count, kArgmaxPerBlock, pv, pi);
    argmax_rows_finish_kernel<<<rows, 256, 0, s>>>(pv, pi, parts, ids);
    return hipGetLastError();
}

}  // namespace qwh

using namespace qwh;

extern "C" {

int32_t qwh_decoder_create(qwh_ctx *ctx, const qwh_decoder_config *config, uint32_t batch, qwh_decoder **out) {
    return qwh_decoder_create_cache(ctx, config, batch, QWH_CACHE_Q8, out);
}

int32_t qwh_decoder_create_cache(qwh_ctx *ctx, const qwh_decoder_config *config, uint32_t batch,
                                 uint32_t cache_format, qwh_decoder **out) {
    if (!ctx || !config || !out || batch == 0) return QWH_E_INVALID_ARGUMENT;
    if (cache_format != QWH_CACHE_F32 && cache_format != QWH_CACHE_Q8)
        return fail(ctx, QWH_E_UNSUPPORTED, "cache format %u is neither f32 (0) nor q8 (1)", cache_format);
    const qwh_decoder_config &c = *config;
    if (c.kv_heads == 0 || c.heads % c.kv_heads != 0)
        return fail(ctx, QWH_E_SHAPE_MISMATCH, "heads %u / kv_heads %u", c.heads, c.kv_heads);
    if (!attention_supported(c.head_dim, c.heads / c.kv_heads))
        return fail(ctx, QWH_E_UNSUPPORTED, "no attention kernel for head_dim %u with %u heads per kv head",
                    c.head_dim, c.heads / c.kv_heads);
    if (c.hidden % 64 || c.ffn % 64 || c.hidden == 0 || c.ffn == 0 || c.layers == 0 || c.vocab == 0)
        return fail(ctx, QWH_E_SHAPE_MISMATCH, "hidden and ffn must be multiples of 64");
    // model.zig:62 position_limit and :1006-1009 validateCapacity.
    if (c.max_positions == 0 || c.max_positions > 8192)
        return fail(ctx, QWH_E_LIMIT_EXCEEDED, "max_positions %u outside 1..8192", c.max_positions);
    qwh_decoder *d = new qwh_decoder();
    d->ctx = ctx;
    d->c = c;
    d->batch = batch;
    d->qw = c.heads * c.head_dim;
    d->kvw = c.kv_heads * c.head_dim;
    d->cache_format = (int32_t)cache_format;
    d->use_graph = getenv("QWH_NO_GRAPH") == nullptr;
    // The kernel plan (plan_step) is made before the first step. Test
    // switches it reads: QWH_DECODER_UNFUSED (separate norm / prep kernels
    // for q4), QWH_DECODER_PER_TOKEN (batch > 1 on the per-token GEMVs),
    // QWH_DECODER_NO_SPLIT (no K-split partial sums).
    auto cleanup = [&](int32_t st) {
        qwh_decoder_destroy(d);
        return st;
    };
    int32_t st = QWH_OK;
    d->layers.resize(c.layers);
    for (uint32_t l = 0; l < c.layers && st == QWH_OK; ++l) {
        qwh_decoder::Layer &L = d->layers[l];
        st = alloc_matrix(d, L.qkv, d->qw + 2 * d->kvw, c.hidden);
        if (st == QWH_OK) st = alloc_matrix(d, L.o, c.hidden, d->qw);
        if (st == QWH_OK) st = alloc_matrix(d, L.gu, 2 * c.ffn, c.hidden);
        if (st == QWH_OK) st = alloc_matrix(d, L.down, c.hidden, c.ffn);
        if (st == QWH_OK) st = dalloc(d, sizeof(float) * c.hidden, reinterpret_cast<void **>(&L.attn_norm));
        if (st == QWH_OK) st = dalloc(d, sizeof(float) * c.hidden, reinterpret_cast<void **>(&L.ffn_norm));
        if (st == QWH_OK) st = dalloc(d, sizeof(float) * c.head_dim, reinterpret_cast<void **>(&L.q_norm));
        if (st == QWH_OK) st = dalloc(d, sizeof(float) * c.head_dim, reinterpret_cast<void **>(&L.k_norm));
        if (st == QWH_OK) st = fill_ones(d, L.attn_norm, c.hidden);
        if (st == QWH_OK) st = fill_ones(d, L.ffn_norm, c.hidden);
        if (st == QWH_OK) st = fill_ones(d, L.q_norm, c.head_dim);
        if (st == QWH_OK) st = fill_ones(d, L.k_norm, c.head_dim);
    }
    if (st == QWH_OK) st = alloc_matrix(d, d->embed, c.vocab, c.hidden);
    if (st == QWH_OK) st = alloc_matrix(d, d->lm_head, c.vocab, c.hidden);
    if (st == QWH_OK) st = dalloc(d, sizeof(float) * c.hidden, reinterpret_cast<void **>(&d->final_norm));
    if (st == QWH_OK) st = fill_ones(d, d->final_norm, c.hidden);
    // RoPE tables.
    std::vector<float> cos_t, sin_t;
    const uint32_t half = c.head_dim / 2;
    build_rope_tables(cos_t, sin_t, half, c.theta, c.max_positions);
    if (st == QWH_OK) st = dalloc(d, cos_t.size() * 4, reinterpret_cast<void **>(&d->rope_cos));
    if (st == QWH_OK) st = dalloc(d, sin_t.size() * 4, reinterpret_cast<void **>(&d->rope_sin));
    if (st == QWH_OK) st = check_hip(ctx, hipMemcpy(d->rope_cos, cos_t.data(), cos_t.size() * 4, hipMemcpyHostToDevice), "rope");
    if (st == QWH_OK) st = check_hip(ctx, hipMemcpy(d->rope_sin, sin_t.data(), sin_t.size() * 4, hipMemcpyHostToDevice), "rope");
    // Caches: per sequence, per layer [scales][codes] (decoder.zig:58-65),
    // or [max_positions][kv_width] f32 (decoder.zig:77-83).
    if (cache_format == QWH_CACHE_Q8) {
        d->cache_scales = (size_t)c.max_positions * (d->kvw / 64) * 2;
        d->cache_codes = (size_t)c.max_positions * d->kvw;
    } else {
        d->cache_scales = 0;
        d->cache_codes = (size_t)c.max_positions * d->kvw * sizeof(float);
    }
    d->layer_stride = d->cache_scales + d->cache_codes;
    d->seq_stride = d->layer_stride * c.layers;
    if (st == QWH_OK) st = dalloc(d, d->seq_stride * batch, reinterpret_cast<void **>(&d->keys));
    if (st == QWH_OK) st = dalloc(d, d->seq_stride * batch, reinterpret_cast<void **>(&d->values));
    if (st == QWH_OK) st = check_hip(ctx, hipMemsetAsync(d->keys, 0, d->seq_stride * batch, ctx->stream), "cache");
    if (st == QWH_OK) st = check_hip(ctx, hipMemsetAsync(d->values, 0, d->seq_stride * batch, ctx->stream), "cache");
    // State.
    d->history_rows = c.max_positions;
    if (st == QWH_OK) st = dalloc(d, 4 * batch, reinterpret_cast<void **>(&d->tokens_dev));
    if (st == QWH_OK) st = dalloc(d, 4 * batch, reinterpret_cast<void **>(&d->pos_dev));
    if (st == QWH_OK) st = dalloc(d, 4 * batch, reinterpret_cast<void **>(&d->hist_base_dev));
    if (st == QWH_OK) st = dalloc(d, 4 * (size_t)batch * d->history_rows, reinterpret_cast<void **>(&d->history_dev));
    if (st == QWH_OK) st = check_hip(ctx, hipMemsetAsync(d->tokens_dev, 0, 4 * batch, ctx->stream), "state");
    if (st == QWH_OK) st = check_hip(ctx, hipMemsetAsync(d->pos_dev, 0, 4 * batch, ctx->stream), "state");
    if (st == QWH_OK) st = check_hip(ctx, hipMemsetAsync(d->hist_base_dev, 0, 4 * batch, ctx->stream), "state");
    if (st == QWH_OK) st = dalloc(d, sizeof(float) * batch * c.hidden, reinterpret_cast<void **>(&d->rows_dev));
    if (st == QWH_OK) st = dalloc(d, 4 * batch, reinterpret_cast<void **>(&d->row_flags_dev));
    if (st == QWH_OK) st = check_hip(ctx, hipMemsetAsync(d->row_flags_dev, 0, 4 * batch, ctx->stream), "state");
    d->pos_host.assign(batch, 0);
    // Scratch.
    const uint32_t widest = c.ffn > c.hidden ? (c.ffn > d->qw ? c.ffn : d->qw) : (c.hidden > d->qw ? c.hidden : d->qw);
    if (st == QWH_OK) st = dalloc(d, sizeof(float) * batch * c.hidden, reinterpret_cast<void **>(&d->hidden));
    if (st == QWH_OK) st = dalloc(d, sizeof(float) * batch * (d->qw + 2 * d->kvw), reinterpret_cast<void **>(&d->qkv));
    if (st == QWH_OK) st = dalloc(d, sizeof(float) * batch * d->qw, reinterpret_cast<void **>(&d->attn));
    if (st == QWH_OK) st = dalloc(d, sizeof(float) * batch * c.ffn, reinterpret_cast<void **>(&d->gu));
    if (st == QWH_OK) st = dalloc(d, sizeof(float) * batch * c.head_dim, reinterpret_cast<void **>(&d->rope_now));
    if (st == QWH_OK) st = dalloc(d, sizeof(float) * batch * (size_t)c.vocab, reinterpret_cast<void **>(&d->logits));
    if (st == QWH_OK) st = dalloc(d, q4_digit_bytes(batch, widest), &d->digits);
    // Batch > 1: digit planes and K-slice partial sums of the matrix-core
    // GEMV (the split plan depends on shapes only, not on q4 / q8).
    if (st == QWH_OK && batch > 1) st = dalloc(d, batch_digit_bytes(batch, widest), &d->batch_digits);
    if (st == QWH_OK && batch > 1) {
        const qwh_decoder::Layer &L0 = d->layers[0];
        size_t parts = 0;
        for (const Matrix *m : {&L0.qkv, &L0.o, &L0.gu, &L0.down, const_cast<const Matrix *>(&d->lm_head)})
            parts = std::max(parts, batch_partial_bytes(batch, *m));
        if (parts) st = dalloc(d, parts, reinterpret_cast<void **>(&d->parts));
    }
    if (st == QWH_OK) st = dalloc(d, sizeof(GenState) + 8 * (size_t)batch, &d->gen);
    AttentionArgs aa{};
    aa.capacity = c.max_positions;
    aa.heads = c.heads;
    aa.kv_heads = c.kv_heads;
    aa.head_dim = c.head_dim;
    aa.batch = batch;
    aa.f32_cache = cache_format == QWH_CACHE_F32;
    d->attn_scratch_bytes = attention_scratch_bytes(ctx->cus, aa);
    if (st == QWH_OK) st = dalloc(d, d->attn_scratch_bytes, &d->attn_scratch);
    d->arg_per_block = kArgmaxPerBlock;
    d->arg_parts = (c.vocab + d->arg_per_block - 1) / d->arg_per_block;
    // Room for either the partial kernel's or the lm_head epilogue's partials.
    const size_t arg_room = (size_t)batch * std::max(d->arg_parts, kGemvMaxPartials);
    if (st == QWH_OK) st = dalloc(d, sizeof(float) * arg_room, reinterpret_cast<void **>(&d->arg_v));
    if (st == QWH_OK) st = dalloc(d, 4 * arg_room, reinterpret_cast<void **>(&d->arg_i));
    if (st == QWH_OK) {
        void *p = nullptr;
        st = check_hip(ctx, hipHostMalloc(&p, 20 * (size_t)batch + sizeof(GenState) + 64, hipHostMallocDefault),
                       "pinned staging");
        d->host_stage = static_cast<uint32_t *>(p);
    }
    if (st == QWH_OK) st = check_hip(ctx, hipStreamSynchronize(ctx->stream), "decoder create");
    if (st != QWH_OK) return cleanup(st);
    *out = d;
    return QWH_OK;
}

int32_t qwh_decoder_destroy(qwh_decoder *d) {
    if (!d) return QWH_E_INVALID_ARGUMENT;
    if (d->ctx) (void)hipStreamSynchronize(d->ctx->stream);
    for (hipGraphExec_t &g : d->graph)
        if (g) (void)hipGraphExecDestroy(g);
    for (void *p : d->allocations) (void)hipFree(p);
    if (d->host_stage) (void)hipHostFree(d->host_stage);
    if (d->pf.host) (void)hipHostFree(d->pf.host);
    delete d;
    return QWH_OK;
}

int32_t qwh_decoder_set_matrix(qwh_decoder *d, uint32_t kind, uint32_t layer, uint64_t handle) {
    if (!d) return QWH_E_INVALID_ARGUMENT;
    const Matrix *m = find_matrix(d->ctx, handle);
    const qwh_decoder_config &c = d->c;
    // The matrix's rows are copied into the decoder's own block, which takes
    // the matrix's format first (ensure_format).
    auto bind = [&](Matrix &dst, uint32_t rows, uint32_t cols, uint32_t offset, uint32_t stride) -> int32_t {
        QWH_TRY(check_matrix(d, m, rows, cols));
        QWH_TRY(ensure_format(d, dst, m->format));
        return copy_rows(d, dst, offset, *m, stride);
    };
    if (kind == QWH_T_EMBED) return bind(d->embed, c.vocab, c.hidden, 0, 1);
    if (kind == QWH_T_LM_HEAD) return bind(d->lm_head, c.vocab, c.hidden, 0, 1);
    if (layer >= c.layers) return fail(d->ctx, QWH_E_INVALID_ARGUMENT, "layer %u of %u", layer, c.layers);
    qwh_decoder::Layer &L = d->layers[layer];
    switch (kind) {
    case QWH_T_Q: return bind(L.qkv, d->qw, c.hidden, 0, 1);
    case QWH_T_K: return bind(L.qkv, d->kvw, c.hidden, d->qw, 1);
    case QWH_T_V: return bind(L.qkv, d->kvw, c.hidden, d->qw + d->kvw, 1);
    case QWH_T_O: return bind(L.o, c.hidden, d->qw, 0, 1);
    case QWH_T_GATE: return bind(L.gu, c.ffn, c.hidden, 0, 2);
    case QWH_T_UP: return bind(L.gu, c.ffn, c.hidden, 1, 2);
    case QWH_T_DOWN: return bind(L.down, c.hidden, c.ffn, 0, 1);
    default: return fail(d->ctx, QWH_E_INVALID_ARGUMENT, "unknown matrix kind %u", kind);
    }
}

int32_t qwh_decoder_set_vector(qwh_decoder *d, uint32_t kind, uint32_t layer, const float *values, uint32_t count) {
    if (!d || !values) return QWH_E_INVALID_ARGUMENT;
    const qwh_decoder_config &c = d->c;
    float *dst = nullptr;
    uint32_t expect = 0;
    if (kind == QWH_T_FINAL_NORM) {
        dst = d->final_norm;
        expect = c.hidden;
    } else {
        if (layer >= c.layers) return fail(d->ctx, QWH_E_INVALID_ARGUMENT, "layer %u of %u", layer, c.layers);
        qwh_decoder::Layer &L = d->layers[layer];
        switch (kind) {
        case QWH_T_ATTN_NORM: dst = L.attn_norm; expect = c.hidden; break;
        case QWH_T_FFN_NORM: dst = L.ffn_norm; expect = c.hidden; break;
        case QWH_T_Q_NORM: dst = L.q_norm; expect = c.head_dim; break;
        case QWH_T_K_NORM: dst = L.k_norm; expect = c.head_dim; break;
        default: return fail(d->ctx, QWH_E_INVALID_ARGUMENT, "unknown vector kind %u", kind);
        }
    }
    if (count != expect) return fail(d->ctx, QWH_E_SHAPE_MISMATCH, "vector of %u values, expected %u", count, expect);
    QWH_TRY(check_hip(d->ctx, hipMemcpy(dst, values, sizeof(float) * count, hipMemcpyHostToDevice), "set vector"));
    return QWH_OK;
}

// f16 bit pattern to f32 on the host (half_float.zig:24-45: exact widening).
static float host_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu;
    float v;
    if (exp == 0x1f) {
        const uint32_t bits = sign | 0x7f800000u | (man << 13);
        std::memcpy(&v, &bits, 4);
        return v;
    }
    v = exp == 0 ? std::ldexp((float)man, -24) : std::ldexp((float)(man | 0x400u), (int)exp - 25);
    return sign ? -v : v;
}

int32_t qwh_decoder_bind_shard(qwh_decoder *d, uint64_t shard, uint32_t flags, uint32_t *bound) {
    if (!d) return QWH_E_INVALID_ARGUMENT;
    qwh_ctx *ctx = d->ctx;
    auto it = ctx->shards.find(shard);
    if (it == ctx->shards.end()) return fail(ctx, QWH_E_NOT_FOUND, "unknown shard handle %llu", (unsigned long long)shard);
    // container.TensorKind (container.zig:337-381): the decoder's tensors are
    // 30..43; layer 0 holds the embedding, final norm and output projection,
    // layer L >= 1 the decoder's layer L - 1.
    const std::vector<qwh_tensor_entry> index = it->second.index;
    uint32_t count = 0;
    for (const qwh_tensor_entry &e : index) {
        if (e.kind < 30 || e.kind > 43 || e.layer >= 1024) continue;  // audio tower, projector
        uint32_t slot = 0xffffffffu, layer = 0;
        bool vector = false;
        if (e.layer == 0) {
            if (e.kind == 30) slot = QWH_T_EMBED;
            else if (e.kind == 32) slot = QWH_T_LM_HEAD;
            else if (e.kind == 31) { slot = QWH_T_FINAL_NORM; vector = true; }
        } else if (e.kind >= 33) {
            if (e.layer > d->c.layers)
                return fail(ctx, QWH_E_SHAPE_MISMATCH, "shard holds decoder layer %u of %u", e.layer, d->c.layers);
            layer = e.layer - 1u;
            static const uint32_t per_layer[11] = {QWH_T_Q, QWH_T_K, QWH_T_V, QWH_T_O, QWH_T_Q_NORM, QWH_T_K_NORM,
                                                   QWH_T_ATTN_NORM, QWH_T_FFN_NORM, QWH_T_GATE, QWH_T_UP, QWH_T_DOWN};
            slot = per_layer[e.kind - 33];
            vector = slot >= QWH_T_ATTN_NORM;
        }
        if (slot == 0xffffffffu) continue;
        if (vector) {
            // A norm weight vector: f32, f16 or bf16 values, widened to f32.
            void *dev = nullptr;
            QWH_TRY(qwh_shard_tensor(ctx, shard, e.kind, e.layer, &dev, nullptr));
            const uint64_t n = e.len_bytes / (e.format == 0 ? 4 : 2);
            std::vector<uint8_t> raw(e.len_bytes);
            QWH_TRY(check_hip(ctx, hipMemcpy(raw.data(), dev, e.len_bytes, hipMemcpyDeviceToHost), "norm download"));
            std::vector<float> values(n);
            for (uint64_t i = 0; i < n; ++i) {
                if (e.format == 0) {
                    std::memcpy(&values[i], &raw[4 * i], 4);
                } else {
                    const uint16_t h = (uint16_t)(raw[2 * i] | (raw[2 * i + 1] << 8));
                    if (e.format == 1) {
                        values[i] = host_f16_to_f32(h);
                    } else {
                        const uint32_t bits = (uint32_t)h << 16;
                        std::memcpy(&values[i], &bits, 4);
                    }
                }
            }
            QWH_TRY(qwh_decoder_set_vector(d, slot, layer, values.data(), (uint32_t)n));
            ++count;
        } else {
            uint64_t m = 0;
            QWH_TRY(qwh_shard_matrix(ctx, shard, e.kind, e.layer, &m));
            int32_t st = qwh_decoder_set_matrix(d, slot, layer, m);
            if (st == QWH_OK && slot == QWH_T_EMBED && (flags & QWH_BIND_OUTPUT_TIED)) {
                st = qwh_decoder_set_matrix(d, QWH_T_LM_HEAD, 0, m);
                if (st == QWH_OK) ++count;
            }
            // The decoder keeps copies: the borrowed handle goes at once.
            const int32_t rel = qwh_matrix_release(ctx, m);
            QWH_TRY(st);
            QWH_TRY(rel);
            ++count;
        }
    }
    QWH_TRY(check_hip(ctx, hipStreamSynchronize(ctx->stream), "bind shard"));
    if (bound) *bound = count;
    return QWH_OK;
}

int32_t qwh_decoder_init_synthetic(qwh_decoder *d, uint32_t seed) {
    return qwh_decoder_init_synthetic_format(d, seed, QWH_FORMAT_Q4);
}

int32_t qwh_decoder_init_synthetic_format(qwh_decoder *d, uint32_t seed, int32_t format) {
    if (!d) return QWH_E_INVALID_ARGUMENT;
    if (format != QWH_FORMAT_Q4 && format != QWH_FORMAT_Q5 && format != QWH_FORMAT_Q8 && !is_dense_format(format))
        return fail(d->ctx, QWH_E_UNSUPPORTED, "synthetic decoder format %d is not f32, f16, q4, q5 or q8", format);
    const qwh_decoder_config &c = d->c;
    QWH_TRY(ensure_format(d, d->embed, format));
    QWH_TRY(ensure_format(d, d->lm_head, format));
    for (qwh_decoder::Layer &L : d->layers)
        for (Matrix *m : {&L.qkv, &L.o, &L.gu, &L.down}) QWH_TRY(ensure_format(d, *m, format));
    const size_t temp_values = (size_t)64 << 20;
    float *temp = nullptr;
    QWH_TRY(check_hip(d->ctx, hipMalloc(&temp, temp_values * 4), "synthetic temp"));
    // Gate and up are generated into a staging matrix, then interleaved.
    Matrix stage;
    stage.format = format;
    stage.rows = c.ffn;
    stage.cols = c.hidden;
    const size_t stage_gpr = (size_t)c.hidden / 64;
    const bool dense = is_dense_format(format);
    int32_t st = dense ? QWH_OK
                       : check_hip(d->ctx, hipMalloc(reinterpret_cast<void **>(&stage.scales), (size_t)c.ffn * stage_gpr * 2),
                                   "synthetic staging");
    if (st == QWH_OK)
        st = check_hip(d->ctx,
                       hipMalloc(reinterpret_cast<void **>(&stage.data),
                                 dense ? (size_t)c.ffn * c.hidden * dense_element_bytes(format)
                                       : (size_t)c.ffn * stage_gpr * (size_t)data_bytes_per_group(format)),
                       "synthetic staging");
    if (st == QWH_OK) st = synth_rows(d, d->embed, 0, c.vocab, seed, kStreamEmbed, 0.02f, temp, temp_values);
    if (st == QWH_OK) st = synth_rows(d, d->lm_head, 0, c.vocab, seed, kStreamLmHead, 0.02f, temp, temp_values);
    for (uint32_t l = 0; l < c.layers && st == QWH_OK; ++l) {
        qwh_decoder::Layer &L = d->layers[l];
        const uint32_t sb = kStreamLayerBase + 16 * l;
        st = synth_rows(d, L.qkv, 0, d->qw, seed, sb + 0, 0.02f, temp, temp_values);
        if (st == QWH_OK) st = synth_rows(d, L.qkv, d->qw, d->kvw, seed, sb + 1, 0.02f, temp, temp_values);
        if (st == QWH_OK) st = synth_rows(d, L.qkv, d->qw + d->kvw, d->kvw, seed, sb + 2, 0.02f, temp, temp_values);
        if (st == QWH_OK) st = synth_rows(d, L.o, 0, c.hidden, seed, sb + 3, 0.02f, temp, temp_values);
        if (st == QWH_OK) st = synth_rows(d, stage, 0, c.ffn, seed, sb + 4, 0.02f, temp, temp_values);
        if (st == QWH_OK) st = copy_rows(d, L.gu, 0, stage, 2);
        if (st == QWH_OK) st = synth_rows(d, stage, 0, c.ffn, seed, sb + 5, 0.02f, temp, temp_values);
        if (st == QWH_OK) st = copy_rows(d, L.gu, 1, stage, 2);
        if (st == QWH_OK) st = synth_rows(d, L.down, 0, c.hidden, seed, sb + 6, 0.02f, temp, temp_values);
    }
    const int32_t sync = check_hip(d->ctx, hipStreamSynchronize(d->ctx->stream), "synthetic model");
    (void)hipFree(temp);
    if (stage.scales) (void)hipFree(stage.scales);
    if (stage.data) (void)hipFree(stage.data);
    return st != QWH_OK ? st : sync;
}

int32_t qwh_decoder_reset(qwh_decoder *d) {
    if (!d) return QWH_E_INVALID_ARGUMENT;
    hipStream_t s = d->ctx->stream;
    QWH_TRY(check_hip(d->ctx, hipMemsetAsync(d->keys, 0, d->seq_stride * d->batch, s), "reset"));
    QWH_TRY(check_hip(d->ctx, hipMemsetAsync(d->values, 0, d->seq_stride * d->batch, s), "reset"));
    QWH_TRY(check_hip(d->ctx, hipMemsetAsync(d->pos_dev, 0, 4 * d->batch, s), "reset"));
    QWH_TRY(check_hip(d->ctx, hipStreamSynchronize(s), "reset"));
    d->pos_host.assign(d->batch, 0);
    return QWH_OK;
}

int32_t qwh_decoder_prefill_random(qwh_decoder *d, uint32_t seq, uint32_t count, uint32_t seed) {
    if (!d || seq >= d->batch) return QWH_E_INVALID_ARGUMENT;
    if (count > d->c.max_positions) return fail(d->ctx, QWH_E_LIMIT_EXCEEDED, "%u positions of %u", count, d->c.max_positions);
    hipStream_t s = d->ctx->stream;
    const size_t values = (size_t)count * d->kvw;
    float *temp = nullptr;
    if (values && d->cache_format == QWH_CACHE_Q8) QWH_TRY(check_hip(d->ctx, hipMalloc(&temp, values * 4), "prefill temp"));
    int32_t st = QWH_OK;
    for (uint32_t l = 0; l < d->c.layers && st == QWH_OK && values; ++l) {
        for (int kv = 0; kv < 2 && st == QWH_OK; ++kv) {
            const uint32_t stream = kStreamCacheBase + 0x100 * seq + 2 * l + kv;
            uint8_t *base = (kv == 0 ? d->keys : d->values) + (size_t)seq * d->seq_stride + (size_t)l * d->layer_stride;
            if (d->cache_format == QWH_CACHE_F32) {
                // The f32 cache holds the rows themselves (decoder.zig:77-83).
                st = check_hip(d->ctx, launch_synth_normal(s, seed, stream, 0, values, 1.0f, reinterpret_cast<float *>(base)),
                               "prefill values");
                continue;
            }
            st = check_hip(d->ctx, launch_synth_normal(s, seed, stream, 0, values, 1.0f, temp), "prefill values");
            if (st == QWH_OK)
                st = check_hip(d->ctx, launch_quantize_rows(s, QWH_FORMAT_Q8, temp, values / 64, base, base + d->cache_scales),
                               "prefill quantize");
        }
    }
    if (st == QWH_OK) {
        d->host_stage[0] = count;
        st = check_hip(d->ctx, hipMemcpyAsync(d->pos_dev + seq, d->host_stage, 4, hipMemcpyHostToDevice, s), "position");
    }
    const int32_t sync = check_hip(d->ctx, hipStreamSynchronize(s), "prefill");
    if (temp) (void)hipFree(temp);
    if (st == QWH_OK && sync == QWH_OK) d->pos_host[seq] = count;
    return st != QWH_OK ? st : sync;
}

int32_t qwh_decoder_cache_planes(qwh_decoder *d, uint32_t seq, uint32_t layer, void **k_scales, void **k_codes,
                                 void **v_scales, void **v_codes) {
    if (!d || seq >= d->batch || layer >= d->c.layers) return QWH_E_INVALID_ARGUMENT;
    uint8_t *kb = d->keys + (size_t)seq * d->seq_stride + (size_t)layer * d->layer_stride;
    uint8_t *vb = d->values + (size_t)seq * d->seq_stride + (size_t)layer * d->layer_stride;
    const bool f32 = d->cache_format == QWH_CACHE_F32;  // no scale planes; the "codes" are f32 rows
    if (k_scales) *k_scales = f32 ? nullptr : kb;
    if (k_codes) *k_codes = kb + d->cache_scales;
    if (v_scales) *v_scales = f32 ? nullptr : vb;
    if (v_codes) *v_codes = vb + d->cache_scales;
    return QWH_OK;
}

int32_t qwh_decoder_position(qwh_decoder *d, uint32_t seq, uint32_t *out) {
    if (!d || !out || seq >= d->batch) return QWH_E_INVALID_ARGUMENT;
    *out = d->pos_host[seq];
    return QWH_OK;
}

int32_t qwh_decoder_set_position(qwh_decoder *d, uint32_t seq, uint32_t position) {
    if (!d || seq >= d->batch) return QWH_E_INVALID_ARGUMENT;
    if (position > d->c.max_positions) return fail(d->ctx, QWH_E_LIMIT_EXCEEDED, "position %u", position);
    d->host_stage[0] = position;
    QWH_TRY(check_hip(d->ctx, hipMemcpyAsync(d->pos_dev + seq, d->host_stage, 4, hipMemcpyHostToDevice, d->ctx->stream), "position"));
    QWH_TRY(check_hip(d->ctx, hipStreamSynchronize(d->ctx->stream), "position"));
    d->pos_host[seq] = position;
    return QWH_OK;
}

// Pinned staging of the generation state: after tokens (batch), row flags
// (batch) and ids (batch), the GenState image followed by done and count.
static GenState *gen_stage(qwh_decoder *d) { return reinterpret_cast<GenState *>(d->host_stage + 3 * (size_t)d->batch); }

// Plain steps (forward, step, generate) run with the stop rules off.
static int32_t plain_mode(qwh_decoder *d) {
    if (d->gen_mode == 0) return QWH_OK;
    GenState *g = gen_stage(d);
    std::memset(g, 0, sizeof(GenState));
    QWH_TRY(check_hip(d->ctx, hipMemcpyAsync(d->gen, g, sizeof(GenState), hipMemcpyHostToDevice, d->ctx->stream),
                      "generation mode"));
    QWH_TRY(check_hip(d->ctx, hipStreamSynchronize(d->ctx->stream), "generation mode"));
    d->gen_mode = 0;
    return QWH_OK;
}

static int32_t upload_tokens(qwh_decoder *d, const uint32_t *tokens, uint32_t steps) {
    for (uint32_t b = 0; b < d->batch; ++b) {
        if (tokens[b] >= d->c.vocab) return fail(d->ctx, QWH_E_SHAPE_MISMATCH, "token %u >= vocab %u", tokens[b], d->c.vocab);
        // decoder.zig:142 PositionExceeded.
        if ((uint64_t)d->pos_host[b] + steps > d->c.max_positions)
            return fail(d->ctx, QWH_E_LIMIT_EXCEEDED, "sequence %u: position %u + %u steps exceeds %u", b,
                        d->pos_host[b], steps, d->c.max_positions);
    }
    QWH_TRY(plain_mode(d));
    memcpy(d->host_stage, tokens, 4 * (size_t)d->batch);
    return check_hip(d->ctx, hipMemcpyAsync(d->tokens_dev, d->host_stage, 4 * (size_t)d->batch, hipMemcpyHostToDevice,
                                            d->ctx->stream), "tokens");
}

int32_t qwh_decoder_forward(qwh_decoder *d, const uint32_t *tokens, int32_t want_logits) {
    if (!d || !tokens) return QWH_E_INVALID_ARGUMENT;
    QWH_TRY(upload_tokens(d, tokens, 1));
    // The history is written only by generate; park its base past any row.
    QWH_TRY(run_step(d, want_logits != 0));
    QWH_TRY(check_hip(d->ctx, hipStreamSynchronize(d->ctx->stream), "forward"));
    for (uint32_t &p : d->pos_host) p += 1;
    return QWH_OK;
}

int32_t qwh_decoder_forward_rows(qwh_decoder *d, const uint32_t *tokens, const float *rows_dev,
                                 const uint8_t *row_mask, int32_t want_logits) {
    if (!d || !tokens || !rows_dev) return QWH_E_INVALID_ARGUMENT;
    QWH_TRY(upload_tokens(d, tokens, 1));
    const uint32_t B = d->batch, H = d->c.hidden;
    uint32_t *flags = d->host_stage + B;
    for (uint32_t b = 0; b < B; ++b) {
        flags[b] = row_mask ? (row_mask[b] != 0) : 1u;
        if (flags[b])
            QWH_TRY(check_hip(d->ctx, hipMemcpyAsync(d->rows_dev + (size_t)b * H, rows_dev + (size_t)b * H,
                                                     sizeof(float) * H, hipMemcpyDeviceToDevice, d->ctx->stream),
                              "audio row"));
    }
    QWH_TRY(check_hip(d->ctx, hipMemcpyAsync(d->row_flags_dev, flags, 4 * (size_t)B, hipMemcpyHostToDevice,
                                             d->ctx->stream), "row flags"));
    const int32_t st = run_step(d, want_logits != 0);
    // Later steps embed their tokens again (outside any captured graph),
    // also when this step failed: no later call may splice stale rows.
    const int32_t clear =
        check_hip(d->ctx, hipMemsetAsync(d->row_flags_dev, 0, 4 * (size_t)B, d->ctx->stream), "row flags");
    QWH_TRY(st);
    QWH_TRY(clear);
    QWH_TRY(check_hip(d->ctx, hipStreamSynchronize(d->ctx->stream), "forward rows"));
    for (uint32_t &p : d->pos_host) p += 1;
    return QWH_OK;
}

namespace {

constexpr uint32_t kPrefillChunk = 256;

// How a prompt runs through the layers:
//   MatrixCores  every layer product has a matrix-core form, o / gate|up /
//                down a K split: int8 digit planes and split GEMVs whose
//                partial sums the next prep adds (prefill_chunk);
//   Rows         every layer matrix has a per-token GEMV that takes the
//                chunk's rows in one launch (f32 / f16 dense, q5 / q8 byte
//                planes, q4 in its fused activation forms): prefill_chunk_rows;
//   Positions    otherwise: the step, one position at a time (batch 1 only).
// The first two also need the attention and the prefill append for the head
// shape.
enum class PrefillForm { MatrixCores, Rows, Positions };

bool rows_gemv_supported(const Matrix &m) {
    if (is_dense_format(m.format)) return gemv_dense_supported(m.format, m.cols);
    if (m.format == QWH_FORMAT_Q4) return gemv_q4_fused_supported(m.rows, m.cols);
    return gemv_b8_supported(m.format, m.rows, m.cols);
}

PrefillForm prefill_form(const qwh_decoder *d) {
    const uint32_t D = d->c.head_dim;
    if (!attention_supported(D, d->c.heads / d->c.kv_heads) || !(D == 64 || D == 128 || D == 256))
        return PrefillForm::Positions;
    bool cores = true, rows = true;
    for (const qwh_decoder::Layer &L : d->layers)
        for (const Matrix *m : {&L.qkv, &L.o, &L.gu, &L.down}) {
            cores = cores && gemv_batch_supported(*m);
            rows = rows && rows_gemv_supported(*m);
        }
    const qwh_decoder::Layer &L0 = d->layers[0];
    if (cores && batch_slices(L0.o) && batch_slices(L0.gu) && batch_slices(L0.down)) return PrefillForm::MatrixCores;
    return rows ? PrefillForm::Rows : PrefillForm::Positions;
}

int32_t prefill_buffers(qwh_decoder *d) {
    qwh_decoder::PrefillBuffers &pf = d->pf;
    if (pf.host) return QWH_OK;
    const qwh_decoder_config &c = d->c;
    const size_t P = kPrefillChunk;
    const uint32_t qkv_n = d->qw + 2 * d->kvw;
    const uint32_t widest = std::max(std::max(c.hidden, c.ffn), d->qw);
    QWH_TRY(dalloc(d, sizeof(float) * P * c.hidden, reinterpret_cast<void **>(&pf.hidden)));
    QWH_TRY(dalloc(d, sizeof(float) * P * qkv_n, reinterpret_cast<void **>(&pf.qkv)));
    QWH_TRY(dalloc(d, sizeof(float) * P * d->qw, reinterpret_cast<void **>(&pf.attn)));
    QWH_TRY(dalloc(d, sizeof(float) * P * c.ffn, reinterpret_cast<void **>(&pf.wide)));
    QWH_TRY(dalloc(d, sizeof(float) * P * c.head_dim, reinterpret_cast<void **>(&pf.rope)));
    QWH_TRY(dalloc(d, batch_digit_bytes((uint32_t)P, widest), &pf.digits));
    const qwh_decoder::Layer &L0 = d->layers[0];
    size_t parts = 4;
    for (const Matrix *m : {&L0.qkv, &L0.o, &L0.gu, &L0.down})
        parts = std::max(parts, batch_partial_bytes((uint32_t)P, *m));
    QWH_TRY(dalloc(d, parts, reinterpret_cast<void **>(&pf.parts)));
    // The attention records: sized per chunk (the range count depends on
    // the chunk's rows and positions), grown by prefill_chunk when a chunk
    // needs more.
    pf.attn_scratch_bytes = 0;
    QWH_TRY(dalloc(d, argmax_scratch_bytes(1, c.vocab), &pf.arg_scratch));
    QWH_TRY(dalloc(d, 3 * 4 * P, reinterpret_cast<void **>(&pf.staged_dev)));
    QWH_TRY(dalloc(d, 4, reinterpret_cast<void **>(&pf.id_dev)));
    void *host = nullptr;
    QWH_TRY(check_hip(d->ctx, hipHostMalloc(&host, 4 * (3 * P + 8), hipHostMallocDefault), "pinned prefill staging"));
    pf.host = static_cast<uint32_t *>(host);
    return QWH_OK;
}

// One row's W * RMSNorm(x) with the batch-1 kernels of the matrix's format.
hipError_t single_row_norm_gemv(qwh_decoder *d, const float *x, const float *norm, const Matrix &w, float *out) {
    hipStream_t s = d->ctx->stream;
    GemvInput in;
    in.mode = GemvInput::RmsNorm;
    in.x = x;
    in.norm = norm;
    in.eps = d->c.eps;
    if (is_dense_format(w.format)) return launch_gemv_dense(s, d->ctx->cus, in, w, 1, out, nullptr);
    if (w.format != QWH_FORMAT_Q4) return launch_gemv_b8(s, d->ctx->cus, in, w, 1, out, nullptr);
    if (gemv_q4_fused_supported(w.rows, w.cols)) return launch_gemv_q4_src(s, d->ctx->cus, in, w, 1, out, nullptr);
    uint32_t *words = static_cast<uint32_t *>(d->digits);
    rmsnorm_digits_kernel<<<1, 256, 0, s>>>(x, norm, w.cols, d->c.eps, words,
                                            reinterpret_cast<float *>(words + (size_t)(w.cols / 32) * dev::kChunkWords));
    GemvInput pre;
    pre.mode = GemvInput::Digits;
    pre.digits = words;
    return launch_gemv_q4_src(s, d->ctx->cus, pre, w, 1, out, nullptr);
}

// Layer l's attention over a chunk's rows (decoder.zig:180-253 for each
// prompt position): the rows are n pseudo-sequences sharing the sequence's
// cache, row i attending to the cache rows below first + i + 1 (its own
// appended first). `query` holds the q | k | v rows, in `slices` planes of
// partial sums when above one; the output goes to pf.attn, and also to
// `digits` as the o projection's activation digits when that is set.
int32_t prefill_attention(qwh_decoder *d, uint32_t seq, uint32_t first, uint32_t n, uint32_t l, const float *query,
                          uint32_t slices, void *digits) {
    qwh_decoder::PrefillBuffers &pf = d->pf;
    const qwh_decoder_config &c = d->c;
    const qwh_decoder::Layer &L = d->layers[l];
    hipStream_t s = d->ctx->stream;
    const uint32_t qkv_n = d->qw + 2 * d->kvw;
    uint8_t *kl = d->keys + (size_t)l * d->layer_stride + (size_t)seq * d->seq_stride;
    uint8_t *vl = d->values + (size_t)l * d->layer_stride + (size_t)seq * d->seq_stride;
    AttentionArgs aa{};
    aa.out = pf.attn;
    aa.query = query;
    aa.query_stride = qkv_n;
    if (slices > 1) {
        aa.query_slices = slices;
        aa.query_plane = (uint64_t)n * qkv_n;
    }
    aa.q_norm = L.q_norm;
    aa.k_norm = L.k_norm;
    aa.rope_now = pf.rope;
    aa.eps = c.eps;
    aa.k_scales = kl;
    aa.k_codes = kl + d->cache_scales;
    aa.v_scales = vl;
    aa.v_codes = vl + d->cache_scales;
    aa.cached_dev = pf.staged_dev + 2 * kPrefillChunk;  // the rows' positions
    aa.cached_bias = 1;
    aa.capacity = first + n;
    aa.heads = c.heads;
    aa.kv_heads = c.kv_heads;
    aa.head_dim = c.head_dim;
    aa.batch = n;
    aa.scale_stride = 0;
    aa.code_stride = 0;
    aa.f32_cache = d->cache_format == QWH_CACHE_F32;
    aa.digits = digits;
    aa.prefill = true;
    const size_t records = attention_scratch_bytes(d->ctx->cus, aa);
    if (records > pf.attn_scratch_bytes) {
        // The previous chunk's kernels may still read the old records.
        QWH_TRY(check_hip(d->ctx, hipStreamSynchronize(s), "prefill scratch"));
        dfree(d, pf.attn_scratch);
        pf.attn_scratch = nullptr;
        pf.attn_scratch_bytes = 0;
        QWH_TRY(dalloc(d, records, &pf.attn_scratch));
        pf.attn_scratch_bytes = records;
    }
    QWH_TRY(check_hip(d->ctx, launch_prefill_append(s, aa, first, n), "prefill cache append"));
    return check_hip(d->ctx, launch_decode_attention_q8(s, d->ctx->cus, aa, pf.attn_scratch, pf.attn_scratch_bytes),
                     "prefill attention");
}

// W * f(x) over a chunk's n rows with the per-token GEMV of w's format
// (rows_gemv_supported): f32 / f16 dense, q5 / q8 byte planes, q4 fused.
hipError_t rows_gemv(qwh_decoder *d, GemvInput::Mode mode, const float *x, const float *norm, const Matrix &w,
                     uint32_t n, float *out, const float *residual, bool pairs) {
    hipStream_t s = d->ctx->stream;
    GemvInput in;
    in.mode = mode;
    in.x = x;
    in.norm = norm;
    in.eps = d->c.eps;
    in.pairs = pairs;
    if (is_dense_format(w.format)) return launch_gemv_dense(s, d->ctx->cus, in, w, n, out, residual);
    if (w.format != QWH_FORMAT_Q4) return launch_gemv_b8(s, d->ctx->cus, in, w, n, out, residual);
    return launch_gemv_q4_src(s, d->ctx->cus, in, w, n, out, residual);
}

// One chunk of a prefill in the Rows form: the prompt rows [c0, c0 + n) at
// positions first .. first + n - 1 through every layer, each projection one
// launch over the chunk's rows (RMSNorm formed in the q|k|v and gate|up
// GEMVs, siluMul in gate|up's epilogue, the residual added by o and down);
// the final hidden rows end in pf.hidden.
int32_t prefill_chunk_rows(qwh_decoder *d, uint32_t seq, uint32_t first, uint32_t n, const float *audio_rows) {
    qwh_decoder::PrefillBuffers &pf = d->pf;
    const qwh_decoder_config &c = d->c;
    hipStream_t s = d->ctx->stream;
    const uint32_t H = c.hidden;
    const uint32_t *tokens_dev = pf.staged_dev, *index_dev = pf.staged_dev + kPrefillChunk;
    embed_prompt_kernel<<<n, 256, 0, s>>>(tokens_dev, index_dev, d->embed.format,
                                          reinterpret_cast<const uint16_t *>(d->embed.scales), d->embed.data, H,
                                          pf.hidden, first, d->rope_cos, d->rope_sin, c.head_dim / 2, pf.rope,
                                          audio_rows);
    QWH_TRY(check_hip(d->ctx, hipGetLastError(), "prefill embedding"));
    for (uint32_t l = 0; l < c.layers; ++l) {
        const qwh_decoder::Layer &L = d->layers[l];
        QWH_TRY(check_hip(d->ctx, rows_gemv(d, GemvInput::RmsNorm, pf.hidden, L.attn_norm, L.qkv, n, pf.qkv, nullptr,
                                            false), "prefill q|k|v"));
        QWH_TRY(prefill_attention(d, seq, first, n, l, pf.qkv, 1, nullptr));
        QWH_TRY(check_hip(d->ctx, rows_gemv(d, GemvInput::F32, pf.attn, nullptr, L.o, n, pf.hidden, pf.hidden, false),
                          "prefill o"));
        QWH_TRY(check_hip(d->ctx, rows_gemv(d, GemvInput::RmsNorm, pf.hidden, L.ffn_norm, L.gu, n, pf.wide, nullptr,
                                            true), "prefill gate|up"));
        QWH_TRY(check_hip(d->ctx, rows_gemv(d, GemvInput::F32, pf.wide, nullptr, L.down, n, pf.hidden, pf.hidden,
                                            false), "prefill down"));
    }
    return QWH_OK;
}

// One chunk of a prefill: prompt rows [c0, c0 + n) of sequence seq at
// positions first .. first + n - 1 through every layer; the last chunk's
// final hidden rows stay in pf.hidden with the last down projection added.
int32_t prefill_chunk(qwh_decoder *d, uint32_t seq, uint32_t first, uint32_t n, const float *audio_rows, bool last) {
    qwh_decoder::PrefillBuffers &pf = d->pf;
    const qwh_decoder_config &c = d->c;
    hipStream_t s = d->ctx->stream;
    const uint32_t H = c.hidden;
    const uint32_t *tokens_dev = pf.staged_dev, *index_dev = pf.staged_dev + kPrefillChunk;
    embed_prompt_kernel<<<n, 256, 0, s>>>(tokens_dev, index_dev, d->embed.format,
                                          reinterpret_cast<const uint16_t *>(d->embed.scales), d->embed.data, H,
                                          pf.hidden, first, d->rope_cos, d->rope_sin, c.head_dim / 2, pf.rope,
                                          audio_rows);
    QWH_TRY(check_hip(d->ctx, hipGetLastError(), "prefill embedding"));
    BatchNorm bn;
    bn.rms = true;
    bn.eps = c.eps;
    PartialSums pending{};
    for (uint32_t l = 0; l < c.layers; ++l) {
        qwh_decoder::Layer &L = d->layers[l];
        GemvInput in;
        in.mode = GemvInput::RmsNorm;
        in.x = pf.hidden;
        in.norm = L.attn_norm;
        in.eps = c.eps;
        QWH_TRY(check_hip(d->ctx, launch_prep_batch(s, in, n, H, pf.digits, &pending), "prefill prep"));
        pending = PartialSums{};
        // K splits chosen for the chunk's token tiles (fewer slices than the
        // step's, each workgroup walking more of K).
        const bool qkv_parts = batch_slices(L.qkv) > 1;
        uint32_t sq = 1;  // planes of q|k|v partial sums in pf.parts (one: the products themselves)
        if (qkv_parts)
            QWH_TRY(check_hip(d->ctx, launch_gemv_batch_parts(s, pf.digits, L.qkv, n, pf.parts, bn, &sq), "prefill q|k|v"));
        else
            QWH_TRY(check_hip(d->ctx, launch_gemv_batch(s, pf.digits, L.qkv, n, pf.qkv, nullptr, false, pf.parts, bn),
                              "prefill q|k|v"));
        QWH_TRY(prefill_attention(d, seq, first, n, l, qkv_parts ? pf.parts : pf.qkv, sq, pf.digits));
        // o, gate|up, down as partial sums, each added by the prep that
        // follows (the batched step's sequence).
        uint32_t so = 0, sgu = 0, sd = 0;
        QWH_TRY(check_hip(d->ctx, launch_gemv_batch_parts(s, pf.digits, L.o, n, pf.parts, BatchNorm{}, &so), "prefill o"));
        GemvInput norm_in;
        norm_in.mode = GemvInput::RmsNorm;
        norm_in.x = pf.hidden;
        norm_in.norm = L.ffn_norm;
        norm_in.eps = c.eps;
        const PartialSums o_sums{pf.parts, so, H, false, pf.hidden};
        QWH_TRY(check_hip(d->ctx, launch_prep_batch(s, norm_in, n, H, pf.digits, &o_sums), "prefill prep"));
        QWH_TRY(check_hip(d->ctx, launch_gemv_batch_parts(s, pf.digits, L.gu, n, pf.parts, bn, &sgu), "prefill gate|up"));
        GemvInput pairs_in;
        pairs_in.mode = GemvInput::F32;
        const PartialSums gu_sums{pf.parts, sgu, 2 * c.ffn, true, nullptr};
        QWH_TRY(check_hip(d->ctx, launch_prep_batch(s, pairs_in, n, c.ffn, pf.digits, &gu_sums), "prefill prep"));
        QWH_TRY(check_hip(d->ctx, launch_gemv_batch_parts(s, pf.digits, L.down, n, pf.parts, BatchNorm{}, &sd),
                          "prefill down"));
        pending = PartialSums{pf.parts, sd, H, false, pf.hidden};
    }
    if (!last) return QWH_OK;  // (only the cache rows of earlier chunks matter)
    // The residual stream after the last layer: the final prep adds the
    // down projection (its digits are not used).
    GemvInput fin;
    fin.mode = GemvInput::RmsNorm;
    fin.x = pf.hidden;
    fin.norm = d->final_norm;
    fin.eps = c.eps;
    return check_hip(d->ctx, launch_prep_batch(s, fin, n, H, pf.digits, &pending), "prefill final");
}

}  // namespace

int32_t qwh_decoder_prefill(qwh_decoder *d, uint32_t seq, const uint32_t *tokens, uint32_t count,
                            uint32_t audio_pad_token, const float *audio_rows_dev, uint32_t audio_steps,
                            uint32_t *next_token) {
    if (!d || !tokens || !next_token || seq >= d->batch) return QWH_E_INVALID_ARGUMENT;
    const qwh_decoder_config &c = d->c;
    // decoder.zig:317: an empty prompt.
    if (count == 0) return fail(d->ctx, QWH_E_SHAPE_MISMATCH, "empty prompt");
    if (audio_steps && !audio_rows_dev) return QWH_E_INVALID_ARGUMENT;
    // decoder.zig:320-331: each audio pad takes the next row, and every row
    // is taken (PromptMismatch otherwise: the reference ABI's shape_mismatch).
    uint32_t pads = 0;
    for (uint32_t i = 0; i < count; ++i) {
        if (tokens[i] >= c.vocab) return fail(d->ctx, QWH_E_SHAPE_MISMATCH, "token %u >= vocab %u", tokens[i], c.vocab);
        if (tokens[i] == audio_pad_token && ++pads > audio_steps)
            return fail(d->ctx, QWH_E_SHAPE_MISMATCH, "more audio pads than the %u audio rows", audio_steps);
    }
    if (pads != audio_steps)
        return fail(d->ctx, QWH_E_SHAPE_MISMATCH, "%u audio pads for %u audio rows", pads, audio_steps);
    const uint32_t pos0 = d->pos_host[seq];
    // decoder.zig:142 PositionExceeded.
    if ((uint64_t)pos0 + count > c.max_positions)
        return fail(d->ctx, QWH_E_LIMIT_EXCEEDED, "position %u + %u prompt tokens exceeds %u", pos0, count,
                    c.max_positions);
    if (!d->planned) QWH_TRY(plan_step(d));
    const PrefillForm form = prefill_form(d);
    if (form == PrefillForm::Positions) {
        // Matrices with neither a matrix-core nor a per-token rows form (a
        // q4 row of an odd K), or a head shape the prefill append does not
        // take: at batch 1 the prompt goes through the step one position at
        // a time, as decoder.zig:319-331 runs it (with more sequences the
        // step would advance them as well).
        if (d->batch != 1)
            return fail(d->ctx, QWH_E_UNSUPPORTED,
                        "prefill of a batch > 1 decoder needs a matrix-core or rows form of every layer matrix");
        uint32_t audio_index = 0;
        for (uint32_t i = 0; i < count; ++i) {
            const uint32_t t = tokens[i];
            const int32_t last = i + 1 == count;
            if (t == audio_pad_token)
                QWH_TRY(qwh_decoder_forward_rows(d, &t, audio_rows_dev + (size_t)audio_index++ * c.hidden, nullptr, last));
            else
                QWH_TRY(qwh_decoder_forward(d, &t, last));
        }
        // decoder.zig:332 argmaxLogits, on the device.
        if (!d->pf.id_dev) QWH_TRY(dalloc(d, 4, reinterpret_cast<void **>(&d->pf.id_dev)));
        QWH_TRY(qwh_argmax_rows(d->ctx, d->logits, 1, c.vocab, d->pf.id_dev));
        QWH_TRY(check_hip(d->ctx, hipMemcpyAsync(d->host_stage, d->pf.id_dev, 4, hipMemcpyDeviceToHost, d->ctx->stream),
                          "prefill id"));
        QWH_TRY(check_hip(d->ctx, hipStreamSynchronize(d->ctx->stream), "prefill"));
        *next_token = d->host_stage[0];
        return QWH_OK;
    }
    QWH_TRY(prefill_buffers(d));
    qwh_decoder::PrefillBuffers &pf = d->pf;
    hipStream_t s = d->ctx->stream;
    uint32_t audio_index = 0;
    for (uint32_t c0 = 0; c0 < count; c0 += kPrefillChunk) {
        const uint32_t n = std::min(kPrefillChunk, count - c0);
        // The pinned staging is reused per chunk: the previous chunk's copy
        // has completed (the stream was synchronized below).
        uint32_t *h_tokens = pf.host, *h_index = pf.host + kPrefillChunk, *h_pos = pf.host + 2 * kPrefillChunk;
        for (uint32_t i = 0; i < n; ++i) {
            const uint32_t t = tokens[c0 + i];
            h_tokens[i] = t;
            h_index[i] = t == audio_pad_token ? audio_index++ : ~0u;
            h_pos[i] = pos0 + c0 + i;
        }
        QWH_TRY(check_hip(d->ctx, hipMemcpyAsync(pf.staged_dev, pf.host, 3 * 4 * (size_t)kPrefillChunk,
                                                 hipMemcpyHostToDevice, s), "prefill tokens"));
        const bool last = c0 + n == count;
        if (form == PrefillForm::MatrixCores) QWH_TRY(prefill_chunk(d, seq, pos0 + c0, n, audio_rows_dev, last));
        else QWH_TRY(prefill_chunk_rows(d, seq, pos0 + c0, n, audio_rows_dev));
        if (last) {
            // decoder.zig:332 argmaxLogits of the last position.
            float *logits = d->logits + (size_t)seq * c.vocab;
            QWH_TRY(check_hip(d->ctx, single_row_norm_gemv(d, pf.hidden + (size_t)(n - 1) * c.hidden, d->final_norm,
                                                           d->lm_head, logits), "prefill lm_head"));
            QWH_TRY(check_hip(d->ctx, launch_argmax_rows(s, logits, 1, c.vocab, pf.arg_scratch, pf.id_dev),
                              "prefill argmax"));
            QWH_TRY(check_hip(d->ctx, hipMemcpyAsync(pf.host + 3 * kPrefillChunk, pf.id_dev, 4, hipMemcpyDeviceToHost, s),
                              "prefill id"));
        }
        QWH_TRY(check_hip(d->ctx, hipStreamSynchronize(s), "prefill"));
    }
    *next_token = pf.host[3 * kPrefillChunk];
    // The sequence's position, also on the device for the steps that follow.
    d->pos_host[seq] = pos0 + count;
    d->host_stage[0] = pos0 + count;
    QWH_TRY(check_hip(d->ctx, hipMemcpyAsync(d->pos_dev + seq, d->host_stage, 4, hipMemcpyHostToDevice, s), "position"));
    return check_hip(d->ctx, hipStreamSynchronize(s), "prefill");
}

int32_t qwh_decoder_step(qwh_decoder *d, const uint32_t *tokens, uint32_t *next_tokens) {
    if (!d || !tokens || !next_tokens) return QWH_E_INVALID_ARGUMENT;
    QWH_TRY(upload_tokens(d, tokens, 1));
    QWH_TRY(run_step(d, true));
    QWH_TRY(check_hip(d->ctx, hipMemcpyAsync(d->host_stage, d->tokens_dev, 4 * (size_t)d->batch, hipMemcpyDeviceToHost,
                                             d->ctx->stream), "next tokens"));
    QWH_TRY(check_hip(d->ctx, hipStreamSynchronize(d->ctx->stream), "step"));
    memcpy(next_tokens, d->host_stage, 4 * (size_t)d->batch);
    for (uint32_t &p : d->pos_host) p += 1;
    return QWH_OK;
}

int32_t qwh_decoder_generate(qwh_decoder *d, const uint32_t *tokens, uint32_t steps, uint32_t *ids_out) {
    if (!d || !tokens || !ids_out) return QWH_E_INVALID_ARGUMENT;
    if (steps == 0) return QWH_OK;
    QWH_TRY(upload_tokens(d, tokens, steps));
    QWH_TRY(check_hip(d->ctx, hipMemcpyAsync(d->hist_base_dev, d->pos_dev, 4 * (size_t)d->batch, hipMemcpyDeviceToDevice,
                                             d->ctx->stream), "history base"));
    for (uint32_t i = 0; i < steps; ++i) QWH_TRY(run_step(d, true));
    QWH_TRY(check_hip(d->ctx, hipMemcpyAsync(ids_out, d->history_dev, 4 * (size_t)d->batch * steps, hipMemcpyDeviceToHost,
                                             d->ctx->stream), "history"));
    QWH_TRY(check_hip(d->ctx, hipStreamSynchronize(d->ctx->stream), "generate"));
    for (uint32_t &p : d->pos_host) p += steps;
    return QWH_OK;
}

int32_t qwh_decoder_generate_until(qwh_decoder *d, const uint32_t *tokens, uint32_t max_tokens,
                                   const uint32_t *stop_tokens, uint32_t stop_count, uint32_t *ids_out,
                                   uint32_t *counts_out) {
    if (!d || !tokens || !counts_out || (max_tokens && !ids_out) || (stop_count && !stop_tokens))
        return QWH_E_INVALID_ARGUMENT;
    if (stop_count > 3) return fail(d->ctx, QWH_E_INVALID_ARGUMENT, "at most 3 stop tokens, got %u", stop_count);
    const uint32_t B = d->batch;
    if (max_tokens > d->history_rows)
        return fail(d->ctx, QWH_E_LIMIT_EXCEEDED, "max_tokens %u exceeds %u", max_tokens, d->history_rows);
    // At most max_tokens - 1 forwards: the last emitted id needs none
    // (decodeStep checks the budget before the next prediction).
    const uint32_t forwards = max_tokens ? max_tokens - 1 : 0;
    QWH_TRY(upload_tokens(d, tokens, forwards));
    GenState *g = gen_stage(d);
    std::memset(g, 0, sizeof(GenState));
    g->mode = 1;
    g->budget = max_tokens;
    g->stop_count = stop_count;
    for (uint32_t i = 0; i < stop_count; ++i) g->stops[i] = stop_tokens[i];
    uint32_t *done = reinterpret_cast<uint32_t *>(g + 1);
    uint32_t *count = done + B;
    uint32_t *row0 = d->host_stage + 2 * (size_t)B;
    bool any = false;
    for (uint32_t b = 0; b < B; ++b) {
        // decodeStep on the caller's next token: a stop token or an empty
        // budget ends the sequence before anything is emitted; else the
        // token is the first id.
        bool stop = max_tokens == 0;
        for (uint32_t i = 0; i < stop_count; ++i) stop = stop || tokens[b] == stop_tokens[i];
        count[b] = stop ? 0u : 1u;
        done[b] = stop || count[b] >= max_tokens ? 1u : 0u;
        row0[b] = tokens[b];
        any = any || !done[b];
    }
    hipStream_t s = d->ctx->stream;
    QWH_TRY(check_hip(d->ctx, hipMemcpyAsync(d->gen, g, sizeof(GenState) + 8 * (size_t)B, hipMemcpyHostToDevice, s),
                      "generation state"));
    if (max_tokens)
        QWH_TRY(check_hip(d->ctx, hipMemcpyAsync(d->history_dev, row0, 4 * (size_t)B, hipMemcpyHostToDevice, s),
                          "first ids"));
    d->gen_mode = 1;
    // Replays in rounds of 16, stopping once every sequence has finished.
    constexpr uint32_t kRound = 16;
    for (uint32_t i = 0; i < forwards && any;) {
        const uint32_t n = std::min(kRound, forwards - i);
        for (uint32_t j = 0; j < n; ++j) QWH_TRY(run_step(d, true));
        i += n;
        if (i >= forwards) break;
        QWH_TRY(check_hip(d->ctx, hipMemcpyAsync(done, static_cast<uint8_t *>(d->gen) + sizeof(GenState), 4 * (size_t)B,
                                                 hipMemcpyDeviceToHost, s), "done flags"));
        QWH_TRY(check_hip(d->ctx, hipStreamSynchronize(s), "done flags"));
        any = false;
        for (uint32_t b = 0; b < B; ++b) any = any || !done[b];
    }
    // Results: counts, ids, and the positions the forwards reached.
    QWH_TRY(check_hip(d->ctx, hipMemcpyAsync(count, static_cast<uint8_t *>(d->gen) + sizeof(GenState) + 4 * (size_t)B,
                                             4 * (size_t)B, hipMemcpyDeviceToHost, s), "counts"));
    if (max_tokens)
        QWH_TRY(check_hip(d->ctx, hipMemcpyAsync(ids_out, d->history_dev, 4 * (size_t)B * max_tokens,
                                                 hipMemcpyDeviceToHost, s), "ids"));
    QWH_TRY(check_hip(d->ctx, hipMemcpyAsync(row0, d->pos_dev, 4 * (size_t)B, hipMemcpyDeviceToHost, s), "positions"));
    QWH_TRY(check_hip(d->ctx, hipStreamSynchronize(s), "generate until"));
    for (uint32_t b = 0; b < B; ++b) {
        counts_out[b] = count[b];
        d->pos_host[b] = row0[b];
        // Rows past a sequence's count hold nothing it emitted.
        for (uint32_t r = count[b]; r < max_tokens; ++r) ids_out[(size_t)r * B + b] = 0;
    }
    return QWH_OK;
}

int32_t qwh_decoder_logits(qwh_decoder *d, uint32_t seq, float *out, uint32_t count) {
    if (!d || !out || seq >= d->batch) return QWH_E_INVALID_ARGUMENT;
    if (count != d->c.vocab) return fail(d->ctx, QWH_E_SHAPE_MISMATCH, "logits count %u, vocab %u", count, d->c.vocab);
    QWH_TRY(check_hip(d->ctx, hipMemcpy(out, d->logits + (size_t)seq * d->c.vocab, 4 * (size_t)count, hipMemcpyDeviceToHost),
                      "logits"));
    return QWH_OK;
}

}  // extern "C"
