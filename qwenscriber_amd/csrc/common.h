// Internal declarations shared by the HIP sources of libqwhip.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/qwhip.h"

namespace qwh {

constexpr int kGroup = 64;          // quant.zig:49
constexpr int kMaxEvents = 256;

inline int data_bytes_per_group(int format) {
    switch (format) {
    case QWH_FORMAT_Q4: return 32;  // quant.zig:53
    case QWH_FORMAT_Q5: return 40;  // quant.zig:56
    case QWH_FORMAT_Q8: return 64;  // quant.zig:59
    default: return 0;
    }
}

// Element formats a Matrix may hold (kernels.zig:160-166: f32, f16).
inline bool is_dense_format(int format) { return format == QWH_FORMAT_F32 || format == QWH_FORMAT_F16; }
inline size_t dense_element_bytes(int format) { return format == QWH_FORMAT_F32 ? 4 : 2; }

inline int format_bias(int format) {  // quant.zig:111-118
    switch (format) {
    case QWH_FORMAT_Q4: return 8;
    case QWH_FORMAT_Q5: return 16;
    case QWH_FORMAT_Q8: return 128;
    default: return 0;
    }
}

struct Matrix {
    int32_t format = 0;
    uint32_t rows = 0;
    uint32_t cols = 0;
    // Quantized formats: rows * cols/64 f16 scales, little endian, row major,
    // and rows * cols/64 * data_bytes_per_group code bytes. f32 / f16: no
    // scale plane, data holds the rows * cols elements, row major.
    uint8_t *scales = nullptr;
    uint8_t *data = nullptr;
    bool owned = false;
    uint64_t shard = 0;         // the shard whose payload it borrows, or 0
};

// A `.qw` shard's payload in device memory and its validated index
// (shard.cpp).
struct Shard {
    void *payload = nullptr;
    uint64_t payload_len = 0;
    std::vector<qwh_tensor_entry> index;
};

// A growable device buffer owned by the context (digit planes, attention
// partials). Growth happens between kernels on the context stream.
struct Workspace {
    void *ptr = nullptr;
    size_t bytes = 0;
};

}  // namespace qwh

struct qwh_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    int cus = 0;
    std::string last_error;
    hipEvent_t events[qwh::kMaxEvents] = {};
    std::unordered_map<uint64_t, qwh::Matrix> matrices;
    std::unordered_map<uint64_t, qwh::Shard> shards;
    uint64_t next_handle = 1;
    qwh::Workspace digits;  // x digit planes for the q4 GEMV
    qwh::Workspace scratch; // attention partials and other per-call scratch
    qwh::Workspace audio;   // audio tower layer / projector activations
    qwh::Workspace front;   // audio front end: chunk planes, flattened steps
    // The audio front end's sinusoidal position table for chunks of
    // front_table_steps steps of front_table_width values (built once per
    // shape on the host, model.zig:751-763).
    qwh::Workspace front_table;
    uint32_t front_table_steps = 0, front_table_width = 0;
};

namespace qwh {

// Records a failure on the context and returns `status`.
int32_t fail(qwh_ctx *ctx, int32_t status, const char *fmt, ...);
// Maps a HIP error to QWH_E_DEVICE with a message, or returns QWH_OK.
int32_t check_hip(qwh_ctx *ctx, hipError_t err, const char *what);
int32_t ensure_workspace(qwh_ctx *ctx, Workspace &ws, size_t bytes);
const Matrix *find_matrix(qwh_ctx *ctx, uint64_t handle);
// Registers a matrix on the context and returns its handle.
uint64_t add_matrix(qwh_ctx *ctx, const Matrix &m);

// ---- kernels launched by the entry points (defined in the .hip files) ----

// Synthetic generator and device quantizer (quantize.hip).
// out[i] = value (first + i) of the stream, times scale, for i < count.
hipError_t launch_synth_normal(hipStream_t s, uint32_t seed, uint32_t stream, uint64_t first,
                               uint64_t count, float scale, float *out);
hipError_t launch_quantize_rows(hipStream_t s, int format, const float *values, uint64_t groups,
                                uint8_t *scales, uint8_t *data);

// q4 activations as signed hex digit planes (gemv.hip).
size_t q4_digit_bytes(uint32_t tokens, uint32_t cols);
hipError_t launch_prep_q4(hipStream_t s, const float *x, uint32_t tokens, uint32_t cols,
                          void *digits);
// The activations a q4 GEMV reads: prepared digit planes, or f32 values the
// kernel encodes itself -- as they are, or after RMSNorm with `norm` / `eps`.
// With `pairs`, rows 2j and 2j+1 of the matrix are a gate row and its up row
// (kernels.zig:233-239 siluMul): the GEMV writes silu(gate_j) * up_j to
// out[t][j] (N/2 values per token) instead of the N products.
struct GemvInput {
    enum Mode { Digits = 0, F32 = 1, RmsNorm = 2, Embed = 4 } mode = Digits;
    const void *digits = nullptr;
    const float *x = nullptr;
    const float *norm = nullptr;
    float eps = 0.0f;
    bool pairs = false;
    // launch_prep_batch, F32 mode only: the values it encodes are
    // gelu(x + bias[col]) (model.zig:866-868) instead of x.
    const float *gelu_bias = nullptr;
    // Embed (q4, K <= 2048): token t's activations are RMSNorm(norm, eps) of
    // row tokens[t] of `embed` (decoder.zig:346-376), or of row t of `rows`
    // where row_flags[t] is set; the row itself is stored to embed_out[t]
    // and the RoPE table row of position pos[t] (rope_half cos, then sin) to
    // rope_now[t].
    const uint32_t *tokens = nullptr;
    const Matrix *embed = nullptr;
    const float *rows = nullptr;
    const uint32_t *row_flags = nullptr;
    float *embed_out = nullptr;
    const uint32_t *pos = nullptr;
    const float *rope_cos = nullptr, *rope_sin = nullptr;
    uint32_t rope_half = 0;
    float *rope_now = nullptr;
    // Optional output (q4 GEMV, no pairs, no residual): argmaxLogits
    // partials of each token's outputs, gemv_q4_partials() per token.
    float *arg_value = nullptr;
    uint32_t *arg_index = nullptr;
};
// Argmax partials per token a q4 GEMV with arg_value leaves (at most 1024).
constexpr uint32_t kGemvMaxPartials = 1024;
uint32_t gemv_q4_partials(int cus, const Matrix &w, const GemvInput &in);
// True when a q4 matrix of this shape has a kernel for the input form
// `mode` (the Embed form takes rows of at most 2048 values).
bool gemv_q4_source_supported(int mode, uint32_t rows, uint32_t cols);
// True when a q4 matrix of this shape has a kernel for the f32 input forms.
bool gemv_q4_fused_supported(uint32_t rows, uint32_t cols);
// y[t][n] (+)= W x; residual may alias out.
hipError_t launch_gemv_q4_src(hipStream_t s, int cus, const GemvInput &in, const Matrix &w,
                              uint32_t tokens, float *out, const float *residual);
hipError_t launch_gemv_q4(hipStream_t s, int cus, const void *digits, const Matrix &w,
                          uint32_t tokens, float *out, const float *residual);
// q5 / q8 GEMV over byte digit planes (quant.zig:253-288 planes) with f32
// activations in the F32 and RmsNorm forms, pairs and residual as the q4
// GEMV; any token count (one launch; each token's workgroups encode its
// activations). Shapes with K <= 6144 and a data plane below 4 GiB; the
// data plane 8-byte (q5) or 16-byte (q8) aligned.
bool gemv_b8_supported(int format, uint32_t rows, uint32_t cols);
hipError_t launch_gemv_b8(hipStream_t s, int cus, const GemvInput &in, const Matrix &w, uint32_t tokens,
                          float *out, const float *residual);
hipError_t launch_gemv_q8(hipStream_t s, int cus, const float *x, const Matrix &w,
                          uint32_t tokens, float *out, const float *residual);

// f16 / f32 weights (gemv_dense.hip, kernels.zig:54-112 linearF32 /
// linearF16): F32 and RmsNorm input forms, pairs and residual as the q4
// GEMV, rows of 1..kDenseMaxCols values (one token's activations in a
// workgroup's 160 KiB of LDS), token counts up to 65535 groups of up to
// four (fewer for wider rows).
constexpr uint32_t kDenseMaxCols = 40956;
bool gemv_dense_supported(int format, uint32_t cols);
hipError_t launch_gemv_dense(hipStream_t s, int cus, const GemvInput &in, const Matrix &w, uint32_t tokens,
                             float *out, const float *residual);
// out[i] = f16 bits of in[i], round to nearest even (half_float.zig:12-16).
hipError_t launch_f32_to_f16(hipStream_t s, const float *in, uint64_t count, uint16_t *out);

// Small-batch q4 / q8 GEMV on the matrix cores (gemv_batch.hip): activations
// as int8 digit planes per 16-token tile, then one MFMA pass over the
// weights. gemv_batch_supported: the matrix has such a form.
size_t batch_digit_bytes(uint32_t tokens, uint32_t cols);
// The partial sums of a split GEMV (launch_gemv_batch_parts) that a prep
// folds into its input: RMSNorm of x + their sum (stored to x_out, which may
// be x), or with pairs (rows = 2 cols) siluMul of the gate / up sums in place
// of x.
struct PartialSums {
    const float *part = nullptr;  // [slices][tokens][rows]
    uint32_t slices = 0, rows = 0;
    bool pairs = false;
    float *x_out = nullptr;
};
hipError_t launch_prep_batch(hipStream_t s, const GemvInput &in, uint32_t tokens, uint32_t cols,
                             void *digits, const PartialSums *sums = nullptr);
// Activations that launch_prep_batch left in RMSNorm form (x * w, without
// the 1 / rms factor): the GEMV applies each token's factor.
struct BatchNorm {
    bool rms = false;
    float eps = 0.0f;
};
// K slices the GEMV splits this shape into (0: no split form, an odd
// number of 64-value groups), and the bytes of partial sums that takes.
uint32_t batch_slices(const Matrix &w);
size_t batch_partial_bytes(uint32_t tokens, const Matrix &w);
bool gemv_batch_supported(const Matrix &w);
// out (+)= W x; with several slices `partials` (batch_partial_bytes) is
// required and a reduce kernel adds them.
hipError_t launch_gemv_batch(hipStream_t s, const void *digits, const Matrix &w, uint32_t tokens,
                             float *out, const float *residual, bool pairs = false, float *partials = nullptr,
                             const BatchNorm &norm = BatchNorm{}, const float *bias = nullptr);
// Up to three matrices of one format, K and split plan, each with a single K
// slice, over the same digits in one launch (out[i] = W_i x); returns
// hipErrorNotSupported, launching nothing, for any other set.
hipError_t launch_gemv_batch_multi(hipStream_t s, const void *digits, const Matrix *const *w, float *const *out,
                                   uint32_t count, uint32_t tokens);
// math.zig:99-116 layerNorm of `tokens` rows of `width` values (width a
// multiple of 64; the statistics of launch_layer_norm) written straight as
// the batch GEMV's activation digits (batch_digit_bytes(tokens, width)).
hipError_t launch_layer_norm_digits(hipStream_t s, const float *x, const float *weight, const float *bias,
                                    uint32_t width, uint32_t tokens, float eps, void *digits);
// Partial sums only: batch_slices(w) planes [slice][token][row], for a prep
// to add (the shape must have a split form). With `slices_used`, the K split
// is chosen for all of the tokens' tiles (never more slices than
// batch_slices(w), so the same buffer holds them) and its slice count is
// returned there for the reader of the partial sums.
hipError_t launch_gemv_batch_parts(hipStream_t s, const void *digits, const Matrix &w, uint32_t tokens,
                                   float *partials, const BatchNorm &norm = BatchNorm{},
                                   uint32_t *slices_used = nullptr);

// q4 / q5 GEMM with bf16 activations (gemm.hip). `scratch` holds the split-K
// partials: gemm_scratch_bytes (0 when the tiles alone fill the device).
size_t gemm_scratch_bytes(int cus, uint32_t tokens, const Matrix &w);
hipError_t launch_gemm_bf16(hipStream_t s, int cus, const uint16_t *x, const Matrix &w,
                            uint32_t tokens, float *out, void *scratch);

// q8 decode attention (attention.hip). `cached` is per sequence when
// cached_dev is non-null (device array of batch values), else uniform.
struct AttentionArgs {
    float *out = nullptr;
    const float *query = nullptr;  // head h of sequence b at query + b * query_stride + h * head_dim
    uint32_t query_stride = 0;     // floats; 0 means heads * head_dim
    uint8_t *k_scales = nullptr, *k_codes = nullptr, *v_scales = nullptr, *v_codes = nullptr;
    uint32_t cached = 0;
    const uint32_t *cached_dev = nullptr;  // optional: positions; cached = value + cached_bias
    uint32_t cached_bias = 0;
    uint32_t capacity = 0;         // upper bound of cached (sizes the grid)
    uint32_t heads = 0, kv_heads = 0, head_dim = 0, batch = 0;
    uint64_t scale_stride = 0, code_stride = 0;  // per sequence, bytes
    // f32 cache (decoder.zig:77-83, kernels.zig:572-627): k_codes / v_codes
    // are [positions][kv_heads * head_dim] f32 planes; no scale planes.
    bool f32_cache = false;
    // Decoder form (q_norm non-null): each query row is the q | k | v
    // projection of the newest position cached - 1. q and k get per-head
    // RMSNorm and RoPE at that position (rope_now: per sequence, that
    // position's table row, head_dim/2 cos then head_dim/2 sin); k and v are
    // appended to the cache.
    const float *q_norm = nullptr, *k_norm = nullptr, *rope_now = nullptr;
    float eps = 0.0f;
    // Optional: the output rows also as the small-batch GEMV's activation
    // digit planes (launch_prep_batch's layout for batch rows of heads *
    // head_dim values), so the output projection needs no separate pass.
    void *digits = nullptr;
    // Optional: the query rows as a K-split GEMV's partial sums (the decoder
    // form's q | k | v projection): query_slices (at most 8) planes of rows,
    // query_plane floats apart, added in slice order as its reduce would.
    uint32_t query_slices = 0;
    uint64_t query_plane = 0;
    // Decoder form for a prefill: every query row's own key / value row is
    // already in the cache (launch_prefill_append), so the range kernels
    // attend to rows below cached including the newest, and the plain merge
    // follows.
    bool prefill = false;
};
// The prefill's cache append (decoder.zig:180-216, :77-105): for query rows
// i < count of one sequence (query_stride apart, optionally as K-slice
// partials), the key row normalized (k_norm) and rotated (rope_now row i),
// key and value stored at cache row first + i (q8 or f32 by f32_cache);
// the cache planes are the sequence's own.
hipError_t launch_prefill_append(hipStream_t s, const AttentionArgs &a, uint32_t first, uint32_t count);
// Head shapes with the range kernels (every form, the decoder's included).
bool attention_supported(uint32_t head_dim, uint32_t ratio);
// Head widths the plain entry points also take for other shapes (any ratio;
// q8: a multiple of 64), through a one-workgroup-per-head kernel.
bool attention_generic_supported(uint32_t head_dim);
// argmaxLogits (decoder.zig:290-301) of `rows` rows of `count` logits into
// ids (the decoder step's kernels); scratch holds argmax_scratch_bytes.
size_t argmax_scratch_bytes(uint32_t rows, uint32_t count);
hipError_t launch_argmax_rows(hipStream_t s, const float *logits, uint32_t rows, uint32_t count, void *scratch,
                              uint32_t *ids);
// Scratch bytes for the range records of either form of the attention.
size_t attention_scratch_bytes(int cus, const AttentionArgs &a);
// Fails with hipErrorInvalidValue, launching nothing, when scratch_bytes
// cannot hold the launch's range records.
hipError_t launch_decode_attention_q8(hipStream_t s, int cus, const AttentionArgs &a,
                                      void *scratch, size_t scratch_bytes);
hipError_t launch_kv_append_q8(hipStream_t s, const float *key, const float *value,
                               uint32_t kv_width, uint32_t position, uint8_t *k_scales,
                               uint8_t *k_codes, uint8_t *v_scales, uint8_t *v_codes);

// Audio convolution front end (frontend.hip). conv3x3Stride2Gelu over
// `batch` images [in_ch][h][w] -> [out_ch][(h-1)/2+1][(w-1)/2+1]; weights
// [out_ch][in_ch][9] f16 bits.
hipError_t launch_conv3x3s2_gelu(hipStream_t s, float *out, const float *in, const uint16_t *weights, const float *bias,
                                 uint32_t batch, uint32_t out_ch, uint32_t in_ch, uint32_t h, uint32_t w);
// The matrix-core form for input channels a multiple of 16 (planes small
// enough for its LDS patch: conv_mfma_supported): weights prepared once per
// weight set into `wprep` (conv_mfma_prep_bytes) by launch_conv_mfma_prep.
bool conv_mfma_supported(uint32_t in_ch, uint32_t h, uint32_t w);
size_t conv_mfma_prep_bytes(uint32_t out_ch, uint32_t in_ch);
hipError_t launch_conv_mfma_prep(hipStream_t s, const uint16_t *weights, uint32_t out_ch, uint32_t in_ch, void *wprep);
hipError_t launch_conv3x3s2_gelu_mfma(hipStream_t s, float *out, const float *in, const void *wprep, const float *bias,
                                     uint32_t batch, uint32_t out_ch, uint32_t in_ch, uint32_t h, uint32_t w);
hipError_t launch_gather_chunks(hipStream_t s, const float *mel, uint32_t bins, uint32_t frames, uint32_t chunk_frames,
                                uint32_t first, uint32_t count, float *out);
hipError_t launch_pack_steps(hipStream_t s, const float *conv3, uint32_t channels, uint32_t bins, uint32_t steps_per_chunk,
                             uint32_t rows, float *flat);
hipError_t launch_add_positions(hipStream_t s, float *rows, const float *table, uint32_t first, uint32_t count,
                                uint32_t width, uint32_t steps_per_chunk);

// Plain streaming read of `bytes` (a multiple of 16, 16-byte aligned) for
// the roofline ceiling (measure.hip); `sink` receives one word per
// workgroup (cus * blocks_per_cu of them).
hipError_t launch_stream_read(hipStream_t s, int cus, const void *src, uint64_t bytes, uint32_t blocks_per_cu,
                              uint32_t *sink);

// Audio tower glue (audio.hip). LayerNorm per token row (out may alias x).
hipError_t launch_layer_norm(hipStream_t s, const float *x, float *out, const float *weight, const float *bias,
                             uint32_t width, uint32_t tokens, float eps);
// x[t][r] + bias[r] (bias may be null): stored to x, GELU of it stored to x,
// or added onto residual[t][r].
enum BiasMode { kBiasAdd = 0, kBiasGelu = 1, kBiasResidual = 2 };
hipError_t launch_bias_epilogue(hipStream_t s, int mode, float *x, const float *bias, float *residual, uint32_t rows,
                                uint32_t tokens);
// Non-causal attention inside windows of window_steps steps starting at
// `first`, the last one ending at `end` (ragged). Row r of q / k / v / out
// starts at ptr + r * stride; head h occupies columns [h * head_dim, (h+1) *
// head_dim). Optional biases are added to q / k / v rows as they are read.
// Strides and base pointers must keep rows 16-byte aligned.
struct AudioAttentionArgs {
    float *out = nullptr;
    const float *q = nullptr, *k = nullptr, *v = nullptr;
    const float *q_bias = nullptr, *k_bias = nullptr, *v_bias = nullptr;
    uint32_t out_stride = 0, q_stride = 0, k_stride = 0, v_stride = 0;
    uint32_t first = 0, end = 0, window_steps = 0;
    uint32_t heads = 0, head_dim = 0;
    float scaling = 0.0f;
};
bool audio_attention_supported(uint32_t head_dim);
hipError_t launch_audio_attention(hipStream_t s, const AudioAttentionArgs &a);

}  // namespace qwh

#define QWH_TRY(expr)                    \
    do {                                 \
        int32_t qwh_status_ = (expr);    \
        if (qwh_status_ != QWH_OK) return qwh_status_; \
    } while (0)
